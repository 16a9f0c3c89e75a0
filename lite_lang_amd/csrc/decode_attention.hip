// Paged GQA decode attention (FlashDecoding split-K), gfx950.
//
// Computes, for every sequence b and query head h,
//   out[b, h] = softmax(q[b,h] . K[slots]^T / sqrt(D)) . V[slots]
// over the first b_seq_len[b] tokens of request row req_to_tokens[b_req_idx[b]].
// Semantics: litelang/kernel/develop_flash_attn/flash_decoding.py:6-312.
//
// Design (differs from the reference on purpose):
//   * one workgroup per (sequence, KV head, split) serves all G = H/KVH query
//     heads of the group, so each K/V row is read from HBM exactly once (the
//     reference launches one program per query head and re-reads it G times);
//   * per 32-token tile a wave computes S^T = K . Q^T and O^T += V^T . P^T on
//     bf16/fp16 MFMA (v_mfma_f32_16x16x32), the G heads padded to 16 columns;
//     K rows are loaded straight from HBM into the MFMA A operand (16 B per
//     lane), V rows go through a padded LDS tile that the A operand of the
//     second product reads transposed;
//   * the split count is fixed per launch and each sequence divides its own
//     length into that many tile-aligned chunks, so short and long sequences
//     are balanced and the grid does not depend on the lengths (graph safe);
//   * the 4 waves of a workgroup merge in LDS; the splits of a (sequence, KV
//     head) are merged by a second, small kernel (log-sum-exp combine of the
//     fp32 partials). An in-launch "last workgroup combines" scheme needs a
//     device-scope release/acquire per workgroup, which on gfx950 writes back
//     and invalidates the whole L2 of the XCD and costs far more than the
//     extra launch.
// A generic VALU path covers fp32 and head dims other than 64/128.
#include "ll_common.h"

namespace {

constexpr int kTile = 32;   // tokens per wave iteration
constexpr int kWaves = 4;   // waves per workgroup
constexpr int kVStride = 136;  // LDS row stride (elements) of the V tile: 272 B, 16 B aligned,
                               // rows 4 apart land 16 banks apart -> conflict-free reads

template <typename T> struct Vec8;
template <> struct Vec8<__bf16> { typedef bf16x8 type; };
template <> struct Vec8<_Float16> { typedef f16x8 type; };

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

struct DecodeArgs {
  const void* q; int64_t q_sb, q_sh;
  const void* k; int64_t k_st, k_sh;
  const void* v; int64_t v_st, v_sh;
  const int32_t* r2t; int64_t r2t_s;
  const void* req_idx; int req64;
  const void* seq_len; int len64;
  void* out; int64_t o_sb, o_sh;
  int B, H, KVH, G;
  int nsplit;
  int units;          // B * KVH
  float scale_log2;   // sm_scale * log2(e)
  float* part_acc;    // [B*H*nsplit, D] unnormalised partial outputs
  float* part_ml;     // [B*H*nsplit, 2] running max (log2 domain) and sum
};

// XCD-aware unit mapping: workgroups are dispatched round-robin over the 8
// XCDs, so all splits of one (sequence, KV head) land on the same XCD.
__device__ __forceinline__ void map_block(int bid, int nsplit, int& unit, int& split) {
  const int xcd = bid & 7;
  const int slot = bid >> 3;
  unit = (slot / nsplit) * 8 + xcd;
  split = slot % nsplit;
}

template <typename T, int D>
__global__ __launch_bounds__(kWaves * 64) void decode_attn_mfma_kernel(DecodeArgs a) {
  typedef typename Vec8<T>::type V8;
  constexpr int DS = D / 32;  // d-steps of 32 for the S^T product
  constexpr int DB = D / 16;  // 16-wide d blocks of the output
  // The V tiles (main loop) and the wave-merge buffers (epilogue) share LDS.
  constexpr int kVtBytes = kWaves * kTile * kVStride * (int)sizeof(T);
  constexpr int kCombBytes = kWaves * 16 * (D + 1) * 4 + 2 * kWaves * 16 * 4;
  __shared__ __attribute__((aligned(16))) char smem[kVtBytes > kCombBytes ? kVtBytes : kCombBytes];
  typedef float CombAcc[16][D + 1];
  CombAcc* comb_acc = (CombAcc*)smem;
  float (*comb_m)[16] = (float (*)[16])(smem + kWaves * 16 * (D + 1) * 4);
  float (*comb_l)[16] = (float (*)[16])(smem + kWaves * 16 * (D + 1) * 4 + kWaves * 16 * 4);

  int unit, split;
  map_block(blockIdx.x, a.nsplit, unit, split);
  if (unit >= a.units) return;
  const int b = unit / a.KVH;
  const int kvh = unit - b * a.KVH;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;  // MFMA column index (query head within the group)
  const int j = lane >> 4;  // lane group (k-slot group)

  const int64_t len = ll_load_idx(a.seq_len, b, a.len64);
  const int64_t rid = ll_load_idx(a.req_idx, b, a.req64);
  const int32_t* slot_row = a.r2t + rid * a.r2t_s;
  const int ntiles = (int)((len + kTile - 1) / kTile);
  const int per_split = (ntiles + a.nsplit - 1) / a.nsplit;
  const int tile_beg = split * per_split;
  const int tile_end = min(ntiles, tile_beg + per_split);

  // Q^T as the B operand: column n = head kvh*G + n, k-slots = d 32*s + 8*j + 0..7
  V8 qb[DS];
  {
    const T* qp = (const T*)a.q + (int64_t)b * a.q_sb + (int64_t)(kvh * a.G + n) * a.q_sh;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      if (n < a.G) {
        qb[s] = *(const V8*)(qp + 32 * s + 8 * j);
      } else {
        for (int e = 0; e < 8; ++e) qb[s][e] = (T)0.f;
      }
    }
  }

  f32x4 acc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max of head n (log2 domain)
  float l_run = 0.f;        // this lane's share of the running sum
  T* vtile = (T*)smem + wave * kTile * kVStride;
  const T* kbase = (const T*)a.k + (int64_t)kvh * a.k_sh;
  const T* vbase = (const T*)a.v + (int64_t)kvh * a.v_sh;

  for (int tile = tile_beg + wave; tile < tile_end; tile += kWaves) {
    const int t0 = tile * kTile;
    // slots of the two 16-token blocks this lane feeds as MFMA rows
    const int tokA = t0 + n, tokB = t0 + 16 + n;
    const bool okA = tokA < len, okB = tokB < len;
    const int slotA = okA ? slot_row[tokA] : 0;
    const int slotB = okB ? slot_row[tokB] : 0;

    // K rows -> A operand of S^T = K . Q^T
    V8 ka[DS], kb[DS];
    const T* kpa = kbase + (int64_t)slotA * a.k_st + 8 * j;
    const T* kpb = kbase + (int64_t)slotB * a.k_st + 8 * j;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      if (okA) ka[s] = *(const V8*)(kpa + 32 * s); else for (int e = 0; e < 8; ++e) ka[s][e] = (T)0.f;
      if (okB) kb[s] = *(const V8*)(kpb + 32 * s); else for (int e = 0; e < 8; ++e) kb[s][e] = (T)0.f;
    }
    // V rows: coalesced 16 B per lane, 16 lanes per row -> LDS tile
    constexpr int VCH = D / 8;            // 16-byte chunks per row
    constexpr int ROWS_PER_LOAD = 64 / VCH;
    V8 vr[kTile / ROWS_PER_LOAD];
#pragma unroll
    for (int i = 0; i < kTile / ROWS_PER_LOAD; ++i) {
      const int r = i * ROWS_PER_LOAD + lane / VCH;
      const int tok = t0 + r;
      // r < 16 is uniform across the wave for a given i
      const int sl = __shfl((r < 16) ? slotA : slotB, r & 15, 64);
      if (tok < len) {
        vr[i] = *(const V8*)(vbase + (int64_t)sl * a.v_st + (lane % VCH) * 8);
      } else {
        for (int e = 0; e < 8; ++e) vr[i][e] = (T)0.f;
      }
    }

    // S^T blocks: rows = tokens 4j+i (block A) and 16+4j+i (block B), column = head n
    f32x4 sA = {0.f, 0.f, 0.f, 0.f}, sB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      sA = mfma16x16x32(ka[s], qb[s], sA);
      sB = mfma16x16x32(kb[s], qb[s], sB);
    }

    // store V tile (after issuing the MFMAs so the loads overlap them)
#pragma unroll
    for (int i = 0; i < kTile / ROWS_PER_LOAD; ++i) {
      const int r = i * ROWS_PER_LOAD + lane / VCH;
      *(V8*)(vtile + r * kVStride + (lane % VCH) * 8) = vr[i];
    }

    // online softmax for head n over this tile's 32 tokens
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = (t0 + 4 * j + i < len) ? sA[i] * a.scale_log2 : -INFINITY;
      x[4 + i] = (t0 + 16 + 4 * j + i < len) ? sB[i] * a.scale_log2 : -INFINITY;
    }
    float tmax = x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, x[i]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);  // finite: token t0 is always valid
    const float alpha = exp2f(m_run - m_new);
    V8 pb;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = exp2f(x[i] - m_new);
      psum += p;
      pb[i] = (T)p;
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int c = 0; c < DB; ++c) acc[c] *= alpha;

    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    // O^T[d, head] += V^T[d, tok] . P^T[tok, head]; k-slot i of lane group j
    // is token 4j+i (i<4) or 16+4j+i-4 (i>=4), matching the S^T layout above.
#pragma unroll
    for (int c = 0; c < DB; ++c) {
      V8 va;
      const T* col = vtile + 16 * c + n;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        va[i] = col[(4 * j + i) * kVStride];
        va[4 + i] = col[(16 + 4 * j + i) * kVStride];
      }
      acc[c] = mfma16x16x32(va, pb, acc[c]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }

  // total sum of head n across the 4 lane groups
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  // ---- merge the waves of this workgroup (the V tiles are dead from here on)
  __syncthreads();
  // acc[c][i] holds O^T[d = 16c + 4j + i][head n]
#pragma unroll
  for (int c = 0; c < DB; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) comb_acc[wave][n][16 * c + 4 * j + i] = acc[c][i];
  if (j == 0) {
    comb_m[wave][n] = m_run;
    comb_l[wave][n] = l_run;
  }
  __syncthreads();

  const int G = a.G;
  const bool direct = (a.nsplit == 1);
  const int64_t pbase = ((int64_t)b * a.H + (int64_t)kvh * G) * a.nsplit + split;
  for (int e = threadIdx.x; e < G * D; e += kWaves * 64) {
    const int g = e / D, d = e - g * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, comb_m[w][g]);
    float L = 0.f, A = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float sc = exp2f(comb_m[w][g] - M);
        L += comb_l[w][g] * sc;
        A += comb_acc[w][g][d] * sc;
      }
    }
    if (direct) {
      T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)(kvh * G + g) * a.o_sh;
      op[d] = ll_from_f32<T>(L > 0.f ? A / L : 0.f);
    } else {
      const int64_t p = pbase + (int64_t)g * a.nsplit;
      a.part_acc[p * D + d] = A;
      if (d == 0) {
        a.part_ml[p * 2] = M;
        a.part_ml[p * 2 + 1] = L;
      }
    }
  }
}

// Log-sum-exp merge of the split partials: one workgroup per (sequence, head).
template <typename T>
__global__ __launch_bounds__(128) void decode_attn_combine_kernel(DecodeArgs a, int D) {
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - b * a.H;
  const int64_t p0 = (int64_t)bh * a.nsplit;
  float M = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.part_ml[(p0 + s) * 2]);
  T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
  for (int d = threadIdx.x; d < D; d += 128) {
    float L = 0.f, A = 0.f;
    if (M != -INFINITY) {
      for (int s = 0; s < a.nsplit; ++s) {
        const float sc = exp2f(a.part_ml[(p0 + s) * 2] - M);
        L += a.part_ml[(p0 + s) * 2 + 1] * sc;
        A += a.part_acc[(p0 + s) * D + d] * sc;
      }
    }
    op[d] = ll_from_f32<T>(L > 0.f ? A / L : 0.f);
  }
}

// ---------------------------------------------------------------- generic path
// One 64-lane workgroup per (sequence, query head); tokens are spread over the
// lanes for q.k, the head dim over the lanes for p.v. Used for fp32 and for
// shapes the MFMA path does not cover; exactness, not speed, is its purpose.
template <typename T>
__global__ __launch_bounds__(64) void decode_attn_generic_kernel(DecodeArgs a, int D, float sm_scale) {
  const int b = blockIdx.y;
  const int h = blockIdx.x;
  const int kvh = h / a.G;
  const int lane = threadIdx.x;
  extern __shared__ float sh[];
  float* qs = sh;             // [D]
  float* ps = sh + D;         // [64]
  int64_t* ss = (int64_t*)(ps + 64);  // [64]
  const int64_t len = ll_load_idx(a.seq_len, b, a.len64);
  const int64_t rid = ll_load_idx(a.req_idx, b, a.req64);
  const T* qp = (const T*)a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  for (int d = lane; d < D; d += 64) qs[d] = ll_to_f32(qp[d]);
  __syncthreads();
  const int nd = (D + 63) / 64;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const T* kb = (const T*)a.k + (int64_t)kvh * a.k_sh;
  const T* vb = (const T*)a.v + (int64_t)kvh * a.v_sh;
  for (int64_t t0 = 0; t0 < len; t0 += 64) {
    const int64_t t = t0 + lane;
    float s = -INFINITY;
    int64_t slot = 0;
    if (t < len) {
      slot = a.r2t[rid * a.r2t_s + t];
      const T* kr = kb + slot * a.k_st;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += qs[d] * (ll_to_f32(kr[d]) * sm_scale);
      s = dot;
    }
    const float cmax = ll_wave_max(s);
    const float mn = fmaxf(m, cmax);
    const float alpha = __expf(m - mn);
    const float p = (t < len) ? __expf(s - mn) : 0.f;
    l = l * alpha + ll_wave_sum(p);
    m = mn;
    ps[lane] = p;
    ss[lane] = slot;
    __syncthreads();
    const int cnt = (int)min((int64_t)64, len - t0);
    for (int r = 0; r < nd; ++r) {
      const int d = lane + 64 * r;
      float v = acc[r] * alpha;
      if (d < D)
        for (int u = 0; u < cnt; ++u) v += ps[u] * ll_to_f32(vb[ss[u] * a.v_st + d]);
      acc[r] = v;
    }
    __syncthreads();
  }
  T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
  for (int r = 0; r < nd; ++r) {
    const int d = lane + 64 * r;
    if (d < D) op[d] = ll_from_f32<T>(l > 0.f ? acc[r] / l : 0.f);
  }
}

int choose_nsplit(int B, int KVH, int64_t max_len) {
  const int units = B * KVH;
  const int64_t tiles = (max_len + kTile - 1) / kTile;
  // aim for ~2 workgroups per CU (256 CUs) while giving each wave >= 1 tile
  int ns = (512 + units - 1) / units;
  const int64_t max_ns = (tiles + kWaves - 1) / kWaves;
  if (ns > max_ns) ns = (int)max_ns;
  if (ns < 1) ns = 1;
  if (ns > 64) ns = 64;
  return ns;
}

}  // namespace

extern "C" int64_t ll_decode_attention_workspace_size(int64_t batch, int64_t q_heads,
                                                      int64_t kv_heads, int64_t head_dim,
                                                      int64_t max_len_in_batch) {
  const int ns = choose_nsplit((int)batch, (int)kv_heads, max_len_in_batch);
  const int64_t parts = batch * q_heads * ns;
  int64_t bytes = ((parts * head_dim * 4 + 255) / 256) * 256;    // partial acc
  bytes += ((parts * 2 * 4 + 255) / 256) * 256;                  // partial (m, l)
  return bytes;
}

extern "C" int ll_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                   const void* k_cache, int64_t k_stride_tok, int64_t k_stride_head,
                                   const void* v_cache, int64_t v_stride_tok, int64_t v_stride_head,
                                   const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                                   const void* b_req_idx, int req_idx_i64, const void* b_seq_len,
                                   int seq_len_i64, void* out, int64_t out_stride_b,
                                   int64_t out_stride_h, int64_t batch, int64_t q_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t max_len_in_batch,
                                   float sm_scale, int dtype, void* workspace,
                                   int64_t workspace_bytes, hipStream_t stream) {
  LL_CHECK_ARG(q && k_cache && v_cache && req_to_tokens && b_req_idx && b_seq_len && out,
               "ll_decode_attention: null pointer");
  LL_CHECK_ARG(kv_heads > 0 && q_heads % kv_heads == 0,
               "ll_decode_attention: q_heads %lld not a multiple of kv_heads %lld",
               (long long)q_heads, (long long)kv_heads);
  LL_CHECK_ARG(head_dim > 0 && head_dim <= 256, "ll_decode_attention: head_dim %lld unsupported",
               (long long)head_dim);
  if (batch == 0) return LL_OK;
  DecodeArgs a;
  a.q = q; a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.k = k_cache; a.k_st = k_stride_tok; a.k_sh = k_stride_head;
  a.v = v_cache; a.v_st = v_stride_tok; a.v_sh = v_stride_head;
  a.r2t = req_to_tokens; a.r2t_s = req_to_tokens_stride;
  a.req_idx = b_req_idx; a.req64 = req_idx_i64;
  a.seq_len = b_seq_len; a.len64 = seq_len_i64;
  a.out = out; a.o_sb = out_stride_b; a.o_sh = out_stride_h;
  a.B = (int)batch; a.H = (int)q_heads; a.KVH = (int)kv_heads; a.G = (int)(q_heads / kv_heads);
  a.units = a.B * a.KVH;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.part_acc = nullptr; a.part_ml = nullptr;

  const bool mfma_ok = (dtype == LL_BF16 || dtype == LL_F16) && (head_dim == 128 || head_dim == 64) &&
                       a.G <= 16 && (q_stride_h % 8 == 0) && (q_stride_b % 8 == 0) &&
                       (k_stride_tok % 8 == 0) && (k_stride_head % 8 == 0) &&
                       (v_stride_tok % 8 == 0) && (v_stride_head % 8 == 0) &&
                       (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0);
  if (!mfma_ok) {
    a.nsplit = 1;
    const size_t shm = head_dim * 4 + 64 * 4 + 64 * 8;
    return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
      hipLaunchKernelGGL((decode_attn_generic_kernel<T>), dim3((unsigned)q_heads, (unsigned)batch),
                         dim3(64), shm, stream, a, (int)head_dim, sm_scale);
      LL_RETURN_LAUNCH();
    });
  }

  a.nsplit = choose_nsplit(a.B, a.KVH, max_len_in_batch);
  if (a.nsplit > 1) {
    const int64_t need = ll_decode_attention_workspace_size(batch, q_heads, kv_heads, head_dim,
                                                            max_len_in_batch);
    LL_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                 "ll_decode_attention: workspace too small (need %lld bytes, got %lld)",
                 (long long)need, (long long)workspace_bytes);
    char* w = (char*)workspace;
    const int64_t parts = batch * q_heads * a.nsplit;
    a.part_acc = (float*)w;
    w += ((parts * head_dim * 4 + 255) / 256) * 256;
    a.part_ml = (float*)w;
  }
  const int groups = (a.units + 7) / 8;
  const unsigned grid = (unsigned)(groups * 8 * a.nsplit);
  if (dtype == LL_BF16) {
    if (head_dim == 128)
      hipLaunchKernelGGL((decode_attn_mfma_kernel<__bf16, 128>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((decode_attn_mfma_kernel<__bf16, 64>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
  } else {
    if (head_dim == 128)
      hipLaunchKernelGGL((decode_attn_mfma_kernel<_Float16, 128>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((decode_attn_mfma_kernel<_Float16, 64>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
  }
  if (a.nsplit > 1) {
    const unsigned cgrid = (unsigned)(batch * q_heads);
    if (dtype == LL_BF16)
      hipLaunchKernelGGL((decode_attn_combine_kernel<__bf16>), dim3(cgrid), dim3(128), 0, stream, a, (int)head_dim);
    else
      hipLaunchKernelGGL((decode_attn_combine_kernel<_Float16>), dim3(cgrid), dim3(128), 0, stream, a, (int)head_dim);
  }
  LL_RETURN_LAUNCH();
}
