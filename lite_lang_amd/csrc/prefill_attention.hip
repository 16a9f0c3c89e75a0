// NoPad varlen causal prefill attention over the paged KV pool, gfx950.
//
// For request b with L = b_seq_len[b] keys (slot row req_to_tokens[b_req_idx[b]])
// and S = shared[b] keys already cached from a previous request, the query
// rows q[b_start_loc[b] + m], m in [0, L - S), attend to keys n <= m + S.
// S = 0 is the plain NoPad prefill. Semantics:
//   litelang/kernel/develop_flash_attn/flash_attn_v2.py:392-566 (no prompt cache)
//   litelang/kernel/develop_flash_attn/flash_attn_v2.py:569-762 (prompt cache)
// including the rounding of the probabilities to the KV dtype before P.V.
//
// Design: one workgroup = 4 waves = 64 query rows of one head; every wave owns
// 16 rows. Per 32-key tile the workgroup stages K and V in LDS once (16 B per
// lane, rows fetched through the slot table) and each wave computes
// S^T = K . Q^T and O^T += V^T . P^T on bf16/fp16 MFMA (v_mfma_f32_16x16x32),
// the same operand arrangement as the decode kernel with query rows in place
// of query heads. Online softmax in the exp2 domain, fp32 state.
#include "ll_common.h"

namespace {

constexpr int kTile = 32;
constexpr int kWaves = 4;
constexpr int kRowsPerWave = 16;
constexpr int kBlockM = kWaves * kRowsPerWave;  // 64 query rows per workgroup
constexpr int kKStride = 136;  // K tile row stride (elements), 16 B aligned
constexpr int kVStride = 136;  // V tile row stride, conflict-free transposed reads

template <typename T> struct Vec8;
template <> struct Vec8<__bf16> { typedef bf16x8 type; };
template <> struct Vec8<_Float16> { typedef f16x8 type; };

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

struct PrefillArgs {
  const void* q; int64_t q_st, q_sh;
  const void* k; int64_t k_st, k_sh;
  const void* v; int64_t v_st, v_sh;
  void* o; int64_t o_st, o_sh;
  const int32_t* r2t; int64_t r2t_s;
  const void* req_idx; int req64;
  const void* start_loc; int start64;
  const void* seq_len; int len64;
  const void* shared; int shared64;
  int H, G;
  int nblk, B, KVH;  // MFMA path: query-row blocks per request, requests, KV heads
  float scale_log2;
  float sm_scale;
};

template <typename T, int D>
__global__ __launch_bounds__(kWaves * 64) void prefill_attn_mfma_kernel(PrefillArgs a) {
  typedef typename Vec8<T>::type V8;
  constexpr int DS = D / 32;
  constexpr int DB = D / 16;
  __shared__ __attribute__((aligned(16))) T ks[2][kTile * kKStride];
  __shared__ __attribute__((aligned(16))) T vs[2][kTile * kVStride];

  // 1-D grid, XCD-aware: workgroups go round-robin over the 8 XCDs, so the G
  // query heads of one (row block, request, KV head) unit take consecutive
  // slots of the same XCD and read its K/V tiles through one L2; the longest
  // (last) row blocks are dispatched first
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int unit = (slot / a.G) * 8 + xcd;
  if (unit >= a.nblk * a.B * a.KVH) return;
  const int kvh = unit % a.KVH;
  const int b = (unit / a.KVH) % a.B;
  const int mblk = a.nblk - 1 - unit / (a.KVH * a.B);
  const int h = kvh * a.G + slot % a.G;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int j = lane >> 4;

  const int64_t L = ll_load_idx(a.seq_len, b, a.len64);
  const int64_t S = a.shared ? ll_load_idx(a.shared, b, a.shared64) : 0;
  const int64_t qlen = L - S;
  const int64_t row0 = (int64_t)mblk * kBlockM;
  if (row0 >= qlen) return;
  const int64_t start = ll_load_idx(a.start_loc, b, a.start64);
  const int64_t rid = ll_load_idx(a.req_idx, b, a.req64);
  const int32_t* slot_row = a.r2t + rid * a.r2t_s;

  // this wave's 16 query rows: m = row0 + 16*wave + n (column n of S^T)
  const int64_t m_row = row0 + kRowsPerWave * wave + n;
  const bool row_ok = m_row < qlen;
  V8 qb[DS];
  {
    const T* qp = (const T*)a.q + (start + (row_ok ? m_row : 0)) * a.q_st + (int64_t)h * a.q_sh;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      if (row_ok) qb[s] = *(const V8*)(qp + 32 * s + 8 * j);
      else for (int e = 0; e < 8; ++e) qb[s][e] = (T)0.f;
    }
  }
  // keys needed by the workgroup: [0, min(L, row0 + 64 + S))
  const int64_t kv_end = min(L, row0 + kBlockM + S);
  // keys needed by this wave's rows: [0, min(L, row0 + 16*wave + 16 + S))
  const int64_t wave_kv_end = min(L, row0 + kRowsPerWave * (wave + 1) + S);

  f32x4 acc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const T* kbase = (const T*)a.k + (int64_t)kvh * a.k_sh;
  const T* vbase = (const T*)a.v + (int64_t)kvh * a.v_sh;
  constexpr int VCH = D / 8;
  constexpr int ROWS_PER_PASS = (kWaves * 64) / VCH;

  // Software pipeline over the 32-key tiles: the K/V rows of tile t+1 and the
  // slot ids of tile t+2 are in flight (registers) while tile t is computed
  // from one of two LDS buffers; one barrier per tile. Loads use clamped
  // addresses (always a valid key) and rows past kv_end are zeroed on the
  // LDS store.
  constexpr int PASSES = (kTile + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
  const int ch = threadIdx.x % VCH, rr = threadIdx.x / VCH;
  int32_t sl_cur[PASSES], sl_nxt[PASSES];
  V8 kreg[PASSES], vreg[PASSES];
  auto load_slots = [&](int64_t t0, int32_t (&s)[PASSES]) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      s[p] = slot_row[min(t0 + p * ROWS_PER_PASS + rr, kv_end - 1)];
  };
  auto load_kv = [&](const int32_t (&s)[PASSES]) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      kreg[p] = *(const V8*)(kbase + (int64_t)s[p] * a.k_st + ch * 8);
      vreg[p] = *(const V8*)(vbase + (int64_t)s[p] * a.v_st + ch * 8);
    }
  };
  load_slots(0, sl_cur);
  load_kv(sl_cur);
  load_slots(kTile, sl_nxt);
  for (int64_t t0 = 0; t0 < kv_end; t0 += kTile) {
    const int buf = (int)((t0 / kTile) & 1);
    T* ksb = ks[buf];
    T* vsb = vs[buf];
    // this tile's rows into LDS (the buffer was last read two tiles ago,
    // before the previous barrier)
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int r = p * ROWS_PER_PASS + rr;
      if (r < kTile) {
        const bool ok = t0 + r < kv_end;
        V8 kv = kreg[p], vv = vreg[p];
        if (!ok)
          for (int e = 0; e < 8; ++e) { kv[e] = (T)0.f; vv[e] = (T)0.f; }
        *(V8*)(ksb + r * kKStride + ch * 8) = kv;
        *(V8*)(vsb + r * kVStride + ch * 8) = vv;
      }
    }
    __syncthreads();
    if (t0 + kTile < kv_end) {
      load_kv(sl_nxt);
      load_slots(t0 + 2 * kTile, sl_nxt);
    }
    if (t0 >= wave_kv_end) continue;  // every row of this wave is causally done

    f32x4 sA = {0.f, 0.f, 0.f, 0.f}, sB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const V8 ka = *(const V8*)(ksb + n * kKStride + 32 * s + 8 * j);
      const V8 kb = *(const V8*)(ksb + (16 + n) * kKStride + 32 * s + 8 * j);
      sA = mfma16x16x32(ka, qb[s], sA);
      sB = mfma16x16x32(kb, qb[s], sB);
    }
    // causal + length mask: key t0+4j+i (A) / t0+16+4j+i (B) vs query row m_row
    const int64_t lim = min(m_row + S, L - 1);  // last key this row may see
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = (t0 + 4 * j + i <= lim) ? sA[i] * a.scale_log2 : -INFINITY;
      x[4 + i] = (t0 + 16 + 4 * j + i <= lim) ? sB[i] * a.scale_log2 : -INFINITY;
    }
    float tmax = x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, x[i]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    // m_new is finite: key 0 is visible to every row and tiles run in order
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
    for (int c = 0; c < DB; ++c) {
      acc[c] *= alpha;
      V8 va;
      const T* col = vsb + 16 * c + n;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        va[i] = col[(4 * j + i) * kVStride];
        va[4 + i] = col[(16 + 4 * j + i) * kVStride];
      }
      acc[c] = mfma16x16x32(va, pb, acc[c]);
    }
  }
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (!row_ok) return;
  T* op = (T*)a.o + (start + m_row) * a.o_st + (int64_t)h * a.o_sh;
  const float inv = 1.0f / l_run;
#pragma unroll
  for (int c = 0; c < DB; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) op[16 * c + 4 * j + i] = ll_from_f32<T>(acc[c][i] * inv);
}

// Generic path: one wave per (query row, head), keys spread over the lanes.
template <typename T>
__global__ __launch_bounds__(64) void prefill_attn_generic_kernel(PrefillArgs a, int D) {
  const int64_t m_row = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int kvh = h / a.G;
  const int lane = threadIdx.x;
  const int64_t L = ll_load_idx(a.seq_len, b, a.len64);
  const int64_t S = a.shared ? ll_load_idx(a.shared, b, a.shared64) : 0;
  if (m_row >= L - S) return;
  const int64_t start = ll_load_idx(a.start_loc, b, a.start64);
  const int64_t rid = ll_load_idx(a.req_idx, b, a.req64);
  extern __shared__ float sh[];
  float* qs = sh;
  float* ps = sh + D;
  int* ss = (int*)(ps + 64);
  const T* qp = (const T*)a.q + (start + m_row) * a.q_st + (int64_t)h * a.q_sh;
  for (int d = lane; d < D; d += 64) qs[d] = ll_to_f32(qp[d]);
  __syncthreads();
  const int64_t kv_end = min(L, m_row + S + 1);
  const int nd = (D + 63) / 64;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const T* kb = (const T*)a.k + (int64_t)kvh * a.k_sh;
  const T* vb = (const T*)a.v + (int64_t)kvh * a.v_sh;
  for (int64_t t0 = 0; t0 < kv_end; t0 += 64) {
    const int64_t t = t0 + lane;
    float s = -INFINITY;
    int slot = 0;
    if (t < kv_end) {
      slot = a.r2t[rid * a.r2t_s + t];
      const T* kr = kb + (int64_t)slot * a.k_st;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += qs[d] * ll_to_f32(kr[d]);
      s = dot * a.scale_log2;
    }
    const float mn = fmaxf(m, ll_wave_max(s));
    const float alpha = exp2f(m - mn);
    const float p = (t < kv_end) ? exp2f(s - mn) : 0.f;
    l = l * alpha + ll_wave_sum(p);
    m = mn;
    ps[lane] = ll_to_f32(ll_from_f32<T>(p));  // P rounded to the KV dtype before P.V
    ss[lane] = slot;
    __syncthreads();
    const int cnt = (int)min((int64_t)64, kv_end - t0);
    for (int r = 0; r < nd; ++r) {
      const int d = lane + 64 * r;
      float v = acc[r] * alpha;
      if (d < D)
        for (int u = 0; u < cnt; ++u) v += ps[u] * ll_to_f32(vb[(int64_t)ss[u] * a.v_st + d]);
      acc[r] = v;
    }
    __syncthreads();
  }
  T* op = (T*)a.o + (start + m_row) * a.o_st + (int64_t)h * a.o_sh;
  for (int r = 0; r < nd; ++r) {
    const int d = lane + 64 * r;
    if (d < D) op[d] = ll_from_f32<T>(acc[r] / l);
  }
}

}  // namespace

extern "C" int ll_prefill_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                                    const void* k_cache, int64_t k_stride_tok,
                                    int64_t k_stride_head, const void* v_cache,
                                    int64_t v_stride_tok, int64_t v_stride_head, void* out,
                                    int64_t out_stride_tok, int64_t out_stride_h,
                                    const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                                    const void* b_req_idx, int req_idx_i64,
                                    const void* b_start_loc, int start_loc_i64,
                                    const void* b_seq_len, int seq_len_i64,
                                    const void* b_shared_seq_len, int shared_i64, int64_t batch,
                                    int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                    int64_t max_input_len, float sm_scale, int dtype,
                                    hipStream_t stream) {
  LL_CHECK_ARG(q && k_cache && v_cache && out && req_to_tokens && b_req_idx && b_start_loc &&
                   b_seq_len,
               "ll_prefill_attention: null pointer");
  LL_CHECK_ARG(kv_heads > 0 && q_heads % kv_heads == 0,
               "ll_prefill_attention: q_heads %lld not a multiple of kv_heads %lld",
               (long long)q_heads, (long long)kv_heads);
  LL_CHECK_ARG(head_dim > 0 && head_dim <= 256 && head_dim % 2 == 0,
               "ll_prefill_attention: head_dim %lld unsupported", (long long)head_dim);
  if (batch == 0 || max_input_len <= 0) return LL_OK;
  PrefillArgs a;
  a.q = q; a.q_st = q_stride_tok; a.q_sh = q_stride_h;
  a.k = k_cache; a.k_st = k_stride_tok; a.k_sh = k_stride_head;
  a.v = v_cache; a.v_st = v_stride_tok; a.v_sh = v_stride_head;
  a.o = out; a.o_st = out_stride_tok; a.o_sh = out_stride_h;
  a.r2t = req_to_tokens; a.r2t_s = req_to_tokens_stride;
  a.req_idx = b_req_idx; a.req64 = req_idx_i64;
  a.start_loc = b_start_loc; a.start64 = start_loc_i64;
  a.seq_len = b_seq_len; a.len64 = seq_len_i64;
  a.shared = b_shared_seq_len; a.shared64 = shared_i64;
  a.H = (int)q_heads; a.G = (int)(q_heads / kv_heads);
  a.sm_scale = sm_scale;
  a.scale_log2 = sm_scale * 1.4426950408889634f;

  const bool mfma_ok = (dtype == LL_BF16 || dtype == LL_F16) && (head_dim == 128 || head_dim == 64) &&
                       (q_stride_tok % 8 == 0) && (q_stride_h % 8 == 0) &&
                       (k_stride_tok % 8 == 0) && (k_stride_head % 8 == 0) &&
                       (v_stride_tok % 8 == 0) && (v_stride_head % 8 == 0) &&
                       (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0);
  if (!mfma_ok) {
    const size_t shm = head_dim * 4 + 64 * 4 + 64 * 4;
    return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
      hipLaunchKernelGGL((prefill_attn_generic_kernel<T>),
                         dim3((unsigned)max_input_len, (unsigned)q_heads, (unsigned)batch), dim3(64),
                         shm, stream, a, (int)head_dim);
      LL_RETURN_LAUNCH();
    });
  }
  a.nblk = (int)ll_cdiv(max_input_len, kBlockM);
  a.B = (int)batch;
  a.KVH = (int)kv_heads;
  const int64_t units = (int64_t)a.nblk * batch * kv_heads;
  const dim3 grid((unsigned)(ll_cdiv(units, 8) * 8 * a.G));
  if (dtype == LL_BF16) {
    if (head_dim == 128)
      hipLaunchKernelGGL((prefill_attn_mfma_kernel<__bf16, 128>), grid, dim3(kWaves * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_attn_mfma_kernel<__bf16, 64>), grid, dim3(kWaves * 64), 0, stream, a);
  } else {
    if (head_dim == 128)
      hipLaunchKernelGGL((prefill_attn_mfma_kernel<_Float16, 128>), grid, dim3(kWaves * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_attn_mfma_kernel<_Float16, 64>), grid, dim3(kWaves * 64), 0, stream, a);
  }
  LL_RETURN_LAUNCH();
}
