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
// Design: one workgroup = 8 waves of 32 query rows, two per SIMD (so that one
// wave's softmax overlaps the other's MFMAs, with the register budget of two
// waves). WPH waves take query rows row0 .. row0 + 32 WPH - 1 of one head and
// the workgroup takes 8 / WPH heads of one KV head (WPH = 2 when the group
// size is a multiple of 4, else 4), so every K/V tile staged in LDS serves 256
// query rows. Per 64-key tile:
//   * K and V rows are DMA'd through the slot table straight into a 4-stage
//     LDS ring (global_load_lds_dwordx4), three tiles ahead of the one being
//     computed, stored key-major with their 16-byte chunks XOR-swizzled by
//     row so that the MFMA operand reads are bank-conflict free; the slot ids
//     are DMA'd too, by every wave into a ring of its own, three tiles ahead
//     of their K/V copies. The P.V operand V^T is read from the key-major V
//     tile with the gfx950 transposing LDS read (ds_read_b64_tr_b16), so no
//     VALU work transposes V;
//   * each wave computes S^T = K . Q^T (2 key blocks of 32, Q^T fragments in
//     registers, v_mfma_f32_32x32x16), the online softmax in the exp2 domain
//     with fp32 state, and O^T += V^T . P^T with P rounded to the KV dtype;
//   * one barrier per tile.
#include <type_traits>

#include "ll_common.h"

namespace {

constexpr int kBK = 64;   // keys per tile
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left free (gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int kVmcntZero = 0x0F70;

constexpr int kStages = 4;  // LDS ring depth (K/V tiles)

// 16 B (4 B) global -> LDS DMA of one lane: lane i of the wave lands at
// lds + 16 i (lds + 4 i).
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 4, 0, 0);
}

// Wait until at most N of this wave's vector memory operations (LDS DMA
// included) are in flight.
template <int N_> __device__ __forceinline__ void vm_wait() {
  static_assert(N_ >= 0 && N_ < 64, "vmcnt is a 6-bit counter");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

// Workgroup barrier for LDS data only: __syncthreads() would also wait for
// every outstanding global access, the copies of the tiles ahead included.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <typename T> struct Vec8;
template <> struct Vec8<__bf16> { typedef bf16x8 type; };
template <> struct Vec8<_Float16> { typedef f16x8 type; };

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
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

template <int D> struct FaGeom {
  static constexpr int ROWB = D * 2;            // bytes of a K or V row
  static constexpr int CH = ROWB / 16;          // 16 B chunks per row
  static constexpr int K_B = kBK * ROWB;        // K tile (V tile the same)
  static constexpr int STAGE_B = 2 * K_B;       // K tile, then V tile
  // LDS chunk position of K chunk c of row r (an involution): the operand
  // reads of 16 lanes (16 rows, one chunk) hit 16 distinct 16 B bank slots
  static __device__ __forceinline__ int kswz(int c, int r) {
    return ROWB == 256 ? (c ^ (r & 15)) : (c ^ ((r >> 1) & 7));
  }
  // LDS chunk position of V chunk c of row (key) r: a transposing read
  // (ds_read_b64_tr_b16) of one P.V fragment touches 8 consecutive keys x 4
  // consecutive chunks; this spreads them over all 16 bank slots of 256 B
  // (each slot twice, the minimum for 512 B)
  static __device__ __forceinline__ int vswz(int c, int r) {
    return ROWB == 256 ? (c ^ ((r & 3) << 2)) : (c ^ (((r >> 1) & 1) << 2));
  }
};


// WPH: waves (of 32 query rows each) per head; the 8 waves of a workgroup
// take 8 / WPH heads of one KV head and 32 * WPH query rows of each
template <int WPH_> struct FaShape {
  static constexpr int WPH = WPH_;
  static constexpr int NW = 8;           // waves per workgroup (two per SIMD)
  static constexpr int HPW = NW / WPH;   // heads per workgroup
  static constexpr int RW = 32;          // query rows per wave
  static constexpr int BQ = WPH * RW;    // query rows of one head per workgroup
};

// The fields of the first loads (lengths, shared prefixes, start offsets,
// request rows and the grid geometry) come as scalar arguments ahead of the
// PrefillArgs block: gfx950 preloads leading scalar kernel arguments into
// SGPRs at dispatch, so those loads do not wait for the argument block's
// load. idx64: bit 0 lengths, 1 shared, 2 starts, 3 request rows are int64.
template <typename T, int D, int WPH>
__global__ __launch_bounds__(512) void prefill_attn_fa_kernel(
    const void* __restrict__ p_len, const void* __restrict__ p_shared,
    const void* __restrict__ p_start, const void* __restrict__ p_rid, int idx64, int nblk, int B,
    int KVH, int G, PrefillArgs a) {
  typedef typename Vec8<T>::type V8;
  typedef FaGeom<D> FG;
  typedef FaShape<WPH> SH;
  constexpr int QB = 1;  // 32-row query blocks per wave
  constexpr int DS = D / 16;  // k-steps of S^T = K . Q^T
  constexpr int DB = D / 32;  // 32-row d blocks of O^T
  constexpr int NT = 64 * SH::NW;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // 1-D grid, XCD-aware: workgroups go round-robin over the 8 XCDs, so the
  // head groups of one (row block, request, KV head) unit take consecutive
  // slots of the same XCD and read its K/V tiles through one L2; the longest
  // (last) row blocks are dispatched first
  const int HP = (G + SH::HPW - 1) / SH::HPW;  // head groups per KV head
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int unit = (slot / HP) * 8 + xcd;
  if (unit >= nblk * B * KVH) return;
  const int hp = slot % HP;
  const int kvh = unit % KVH;
  const int b = (unit / KVH) % B;
  const int mblk = nblk - 1 - unit / (KVH * B);
  // every per-request value in one round trip (the start and the request
  // row too, although a workgroup past its request's rows does not use them)
  const int64_t L = ll_load_idx(p_len, b, idx64 & 1);
  const int64_t S = p_shared ? ll_load_idx(p_shared, b, (idx64 >> 1) & 1) : 0;
  const int64_t start = ll_load_idx(p_start, b, (idx64 >> 2) & 1);
  const int64_t rid = ll_load_idx(p_rid, b, (idx64 >> 3) & 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, hf = lane >> 5;
  const int gh = SH::HPW * hp + wave / SH::WPH;  // head within the KV head's group
  const bool head_ok = gh < G;
  const int h = kvh * G + (head_ok ? gh : 0);

  const int64_t qlen = L - S;
  const int64_t blk0 = (int64_t)mblk * SH::BQ;
  if (blk0 >= qlen) return;
  const int32_t* slot_row = a.r2t + rid * a.r2t_s;
  // token indices within a request fit in 32 bits (lengths below 2^31)
  const int row0 = (int)blk0 + SH::RW * (wave % SH::WPH);  // this wave's first query row
  const bool wave_ok = head_ok && row0 < qlen;
  const int kv_end = (int)min(L, blk0 + SH::BQ + S);     // keys of the workgroup
  const int wave_kv_end = (int)min(L, (int64_t)row0 + SH::RW + S);  // keys of this wave's rows
  const int Si = (int)S, Lm1 = (int)L - 1, qlast = (int)qlen - 1;

  // Q^T fragments (B operand: column = query row row0 + l32, clamped into the
  // request; k-slots = d 16 s + 8 hf .. +7), in registers for the whole loop
  V8 qreg[DS];
  {
    const int r = min(row0 + l32, qlast);
    const T* qp = (const T*)a.q + (start + r) * a.q_st + (int64_t)h * a.q_sh + 8 * hf;
#pragma unroll
    for (int s = 0; s < DS; ++s) qreg[s] = *(const V8*)(qp + 16 * s);
  }

  // K and V tiles go from the pool straight into an NST-stage LDS ring
  // (global_load_lds_dwordx4, no VGPR staging); the slot ids that address
  // them are DMA'd likewise, by every wave into a ring of its own, NST - 1
  // tiles before the tile's K/V copies. Per loop iteration t every wave
  // issues one group: its K/V copies of tile t + NST - 1 (when that tile
  // exists) and its slot ids of tile t + 2 NST - 2 (clamped, always), so
  // that NST - 1 tiles are in flight while tile t is computed.
  const T* kbase = (const T*)a.k + (int64_t)kvh * a.k_sh;
  const T* vbase = (const T*)a.v + (int64_t)kvh * a.v_sh;
  constexpr int NST = kStages;
  constexpr int RPI = 64 / FG::CH;                     // rows per DMA instruction
  constexpr int IPW = kBK * FG::ROWB / 1024 / SH::NW;  // K (and V) instructions per wave per tile
  constexpr int KVC = 2 * IPW;                         // K and V
  static_assert(IPW >= 1 && IPW * SH::NW * 1024 == kBK * FG::ROWB, "tile rows over the waves");
  char* wslots = smem + NST * FG::STAGE_B + wave * (NST * kBK * 4);
  const int ntiles = (kv_end + kBK - 1) / kBK;
  auto slot_copy = [&](int u) {  // slot ids of keys 64 u + lane (clamped) -> ring entry u % NST
    dma4(slot_row + min(u * kBK + lane, kv_end - 1), wslots + (u % NST) * (kBK * 4));
  };
  const int dr = lane / FG::CH, dp = lane % FG::CH;
  auto kv_copy = [&](int u) {  // this wave's K and V rows of tile u -> stage u % NST
    char* kl = smem + (u % NST) * FG::STAGE_B;
    char* vl = kl + FG::K_B;
    const int32_t* sl = (const int32_t*)(wslots + (u % NST) * (kBK * 4));
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int ii = wave * IPW + i;
      const int r = ii * RPI + dr;  // the LDS chunk position dp of row r holds chunk swz(dp, r)
      const int64_t slot = sl[r];
      dma16(kbase + slot * a.k_st + 8 * FG::kswz(dp, r), kl + ii * 1024);
      dma16(vbase + slot * a.v_st + 8 * FG::vswz(dp, r), vl + ii * 1024);
    }
  };
  // at the top of iteration t only the groups of iterations t-NST+2 .. t-1
  // may be in flight: NST - 2 slot copies and the K/V copies of the `later`
  // tiles among t+1 .. t+NST-2 that exist
  auto wait_tile = [&](int later) {
    static_assert(NST == 3 || NST == 4, "waits below are written for 3 or 4 stages");
    if (NST == 4 && later >= 2) vm_wait<(NST - 2) + 2 * KVC>();
    else if (later >= 1) vm_wait<(NST - 2) + KVC>();
    else vm_wait<NST - 2>();
  };

  f32x16 acc[DB][QB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) acc[db][qb] = (f32x16){};
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
  }

  // slot ids of tiles 0 .. NST-2, then (every load so far landed, Q
  // fragments included: a real s_waitcnt, which the compiler's own wait
  // insertion accounts for, so that it waits for none of them in the loop)
  // the groups of iterations -NST+1 .. -1
#pragma unroll
  for (int u = 0; u < NST - 1; ++u) slot_copy(u);
  __builtin_amdgcn_s_waitcnt(kVmcntZero);
#pragma unroll
  for (int u = 0; u < NST - 1; ++u) {
    if (u < ntiles) kv_copy(u);
    slot_copy(u + NST - 1);
  }

  // S^T[key 32 kb + 8 g + 4 hf + i][query 32 qb + l32] of the current tile in
  // sacc[kb][qb][4 g + i]; the row maxima it proposes in m_cand
  f32x16 sacc[2][QB];
  float m_cand[QB];
  auto scores = [&](int t0, int buf) {
    const char* kl = smem + buf * FG::STAGE_B;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sacc[kb][qb] = (f32x16){};
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      V8 qf[QB], ka[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int r = 32 * x + l32;
        ka[x] = *(const V8*)(kl + r * FG::ROWB + FG::kswz(2 * s + hf, r) * 16);
      }
      qf[0] = qreg[s];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[kb][qb] = mfma32(ka[kb], qf[qb], sacc[kb][qb]);
    }
    // the causal + length mask only where a key can pass the wave's first
    // row's limit (masked keys -> -inf), then the tile's row maxima in the
    // exp2 domain (finite: key 0 is visible to every row, scale_log2 > 0)
    const bool need_mask = t0 + kBK - 1 > min(row0 + Si, Lm1);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (need_mask) {
        // last key this row sees, relative to the tile (rows past the
        // request see every key of it)
        const int lim = min(row0 + 32 * qb + l32 + Si, Lm1) - t0;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = 32 * kb + 8 * (e >> 2) + 4 * hf + (e & 3);
            if (key > lim) sacc[kb][qb][e] = -INFINITY;
          }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sacc[kb][qb][e]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      m_cand[qb] = fmaxf(m_run[qb], tmax * a.scale_log2);
    }
  };
  // p = 2^(s * scale_log2 - m_run) rounded to T as the P^T fragments of the 4
  // key steps (step s = keys 16 s + {4hf..4hf+3, 8+4hf..8+4hf+3}: S^T block
  // kb = s / 2, g = 2 (s % 2) and g + 1), the row sums into l_run, then
  // O^T[d 32 db + 8 g + 4 hf + i][query 32 qb + l32] += V^T . P^T
  // V^T fragment of key step s, d block db (A operand: lane -> d = 32 db +
  // l32, k-slots 8 hf .. 8 hf + 7 = keys 16 s + 4 hf + {0..3} and
  // 16 s + 8 + 4 hf + {0..3}, the order of the P^T fragments): two
  // transposing reads, the 16-lane group g = lane / 16 reading keys
  // 16 s + 4 (g / 2) + j / 4 (+ 8), d 32 db + 16 (g % 2) + 4 (j % 4) .. + 3
  const int tg = lane >> 4, tj = lane & 15;
  // the two transposing reads of fragment (s, db): keys 16 s + 4 (g / 2) + j / 4
  // and 8 keys further, d bytes 64 db + 32 (g % 2) + 8 (j % 4)
  auto vfrag_reads = [&](const char* vl, int s, int db, s16x4& lo, s16x4& hi) {
    const int key = 16 * s + 4 * (tg >> 1) + (tj >> 2);
    const int dbyte = 64 * db + 32 * (tg & 1) + 8 * (tj & 3);
    const int c = dbyte >> 4, off = dbyte & 15;
    lo = ll_lds_read_tr16(vl + key * FG::ROWB + FG::vswz(c, key) * 16 + off);
    hi = ll_lds_read_tr16(vl + (key + 8) * FG::ROWB + FG::vswz(c, key + 8) * 16 + off);
  };
  auto accumulate = [&](int buf) {
    const char* vl = smem + buf * FG::STAGE_B + FG::K_B;
    V8 pf[QB][4];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float psum = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int kb = s >> 1, e0 = 8 * (s & 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float p = __builtin_amdgcn_exp2f(
              __builtin_fmaf(sacc[kb][qb][e0 + e], a.scale_log2, -m_run[qb]));
          psum += p;
          pf[qb][s][e] = (T)p;
        }
      }
      psum += __shfl_xor(psum, 32, 64);
      l_run[qb] += psum;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      s16x4 vr[2 * DB];  // lo, hi of each d block
#pragma unroll
      for (int db = 0; db < DB; ++db) vfrag_reads(vl, s, db, vr[2 * db], vr[2 * db + 1]);
      ll_lds_wait_tie(vr);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const V8 va = __builtin_bit_cast(
            V8, __builtin_shufflevector(vr[2 * db], vr[2 * db + 1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) acc[db][qb] = mfma32(va, pf[qb][s], acc[db][qb]);
      }
    }
  };
  for (int t = 0; t < ntiles; ++t) {
    wait_tile(min(NST - 2, ntiles - 1 - t));
    // every wave's copies of tile t are in; every wave is done with tile
    // t - 1, whose stage the copies of tile t + NST - 1 refill
    lds_barrier();
    if (t + NST - 1 < ntiles) kv_copy(t + NST - 1);
    slot_copy(t + 2 * NST - 2);
    const int t0 = t * kBK, buf = t % NST;
    if (wave_ok && t0 < wave_kv_end) {
      scores(t0, buf);
      // running maxima; the output rows are rescaled when a row's max rises
      // (every lane of a block skips the multiply when none does)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_cand[qb]);
        m_run[qb] = m_cand[qb];
        l_run[qb] *= alpha;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
          for (int db = 0; db < DB; ++db) acc[db][qb] *= alpha;
        }
      }
      accumulate(buf);
    }
  }
  // no copy may still be writing this workgroup's LDS when it ends
  vm_wait<0>();
  if (!wave_ok) return;
  // acc[db][qb][4 g + i] = O^T[d = 32 db + 8 g + 4 hf + i][query row0 + 32 qb + l32]
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int r = row0 + 32 * qb + l32;
    if (r > qlast) continue;
    const float inv = 1.0f / l_run[qb];
    T* op = (T*)a.o + (start + r) * a.o_st + (int64_t)h * a.o_sh + 4 * hf;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef T T4 __attribute__((ext_vector_type(4)));
        T4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = ll_from_f32<T>(acc[db][qb][4 * g + i] * inv);
        *(T4*)(op + 32 * db + 8 * g) = y;
      }
  }
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
  // four heads of 64 rows per workgroup when the group size allows, else two
  // heads of 128 rows (fewer idle head slots for G = 6 or 7)
  const int wph = (a.G % 4 == 0) ? 2 : 4;
  a.nblk = (int)ll_cdiv(max_input_len, 32 * wph);
  a.B = (int)batch;
  a.KVH = (int)kv_heads;
  const int64_t units = (int64_t)a.nblk * batch * kv_heads;
  const dim3 grid((unsigned)(ll_cdiv(units, 8) * 8 * ll_cdiv(a.G, 8 / wph)));
  const dim3 block(512);
  auto launch = [&](auto tag, auto dtag) {
    typedef decltype(tag) T;
    constexpr int D = decltype(dtag)::value;
    constexpr size_t lds = kStages * FaGeom<D>::STAGE_B + 8 * kStages * kBK * 4;
    const int idx64 = (a.len64 ? 1 : 0) | (a.shared64 ? 2 : 0) | (a.start64 ? 4 : 0) |
                      (a.req64 ? 8 : 0);
    if (wph == 2)
      hipLaunchKernelGGL((prefill_attn_fa_kernel<T, D, 2>), grid, block, lds, stream, a.seq_len,
                         a.shared, a.start_loc, a.req_idx, idx64, a.nblk, a.B, a.KVH, a.G, a);
    else
      hipLaunchKernelGGL((prefill_attn_fa_kernel<T, D, 4>), grid, block, lds, stream, a.seq_len,
                         a.shared, a.start_loc, a.req_idx, idx64, a.nblk, a.B, a.KVH, a.G, a);
  };
  typedef std::integral_constant<int, 128> D128;
  typedef std::integral_constant<int, 64> D64;
  if (dtype == LL_BF16) {
    if (head_dim == 128) launch(__bf16{}, D128{}); else launch(__bf16{}, D64{});
  } else {
    if (head_dim == 128) launch(_Float16{}, D128{}); else launch(_Float16{}, D64{});
  }
  LL_RETURN_LAUNCH();
}
