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
//   * the split's slot ids are staged in LDS first; then every wave streams
//     the K and V rows of its own 16-token tiles straight into LDS with
//     global_load_lds_dwordx4 (no VGPR staging, 16 B chunks XOR-swizzled per
//     row), two tiles in flight per wave, with no workgroup barrier in the
//     token loop -- the kernel is bound by how many bytes are in flight;
//   * per tile S^T = K . Q^T on v_mfma_f32_16x16x32 (the G heads padded to 16
//     columns) and O^T += V^T . P^T on v_mfma_f32_16x16x16, whose B operand
//     is exactly the S^T accumulator layout, so P never leaves registers; P
//     enters as a high and a low part in the KV dtype (two MFMAs), keeping
//     the reference's fp32 probabilities to ~2^-17 instead of rounding them;
//   * the split count is fixed per launch and each sequence divides its own
//     length into that many tile-aligned chunks, so the grid does not depend
//     on the lengths (graph safe);
//   * the 8 waves merge in LDS; the splits of a (sequence, KV head) are merged
//     by its last split (the workgroup with the unit's highest index), which
//     polls the others' partial words in the XCD's L2 (all splits of a unit
//     run on one XCD) while it merges its own waves: no ticket, and no wait
//     for stores to be acknowledged, on the way to the output (a device-scope
//     version was measured slower than a second launch). The quantising
//     variant (one sequence's heads span units on different XCDs) merges in
//     the last workgroup of the sequence to take a ticket, and batches
//     beyond kMergeUnits units in a second kernel.
// A generic VALU path covers fp32 and head dims other than 64/128.
#include "ll_common.h"

#include <atomic>
#include <mutex>

namespace {

constexpr int kTT = 16;     // tokens per tile
constexpr int kWaves = 8;   // waves per split-stage workgroup
constexpr int kCombWaves = 4;  // waves (one (sequence, head) each) per combine workgroup
constexpr int kRing = 2;    // tile buffers per wave
constexpr int kUnitMergeSplits = 8;  // splits the per-unit merge holds in registers
constexpr int kUnitMergeSpin = 1 << 20;  // default polls before the per-unit merge gives up
                                         // (never reached: the words are already on their way)

template <typename T> struct Vec8;
template <> struct Vec8<__bf16> { typedef bf16x8 type; };
template <> struct Vec8<_Float16> { typedef f16x8 type; };
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
template <typename T> struct Vec4;
template <> struct Vec4<__bf16> { typedef s16x4 type; };
template <> struct Vec4<_Float16> { typedef f16x4 type; };

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ s16x4 as_v4(s16x4 x, s16x4) { return x; }
__device__ __forceinline__ f16x4 as_v4(s16x4 x, f16x4) { return __builtin_bit_cast(f16x4, x); }

// raw 16-bit pattern of an element (the 16x16x16 bf16 operands are short vectors)
__device__ __forceinline__ short bits16(__bf16 x) { return __builtin_bit_cast(short, x); }
__device__ __forceinline__ _Float16 bits16(_Float16 x) { return x; }

// 16 B global -> LDS DMA of one lane (lane i of the wave lands at lds + 16 i).
// Kept out of the kernel templates: a dependent call of this device-only
// builtin makes the host pass drop the template's launch stub.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

// Workgroup barrier for LDS data only: __syncthreads() also waits for every
// outstanding global access (vmcnt(0)), which would drain the K/V copies in
// flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int N_> __device__ __forceinline__ void vm_wait() {
  static_assert(N_ >= 0 && N_ < 64, "vmcnt is a 6-bit counter");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
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
  int max_len;        // tokens beyond it are ignored (as the reference's grid does)
  int slots_cap;      // slot entries the LDS slot table holds (>= tiles per split * 16)
  float scale_log2;   // sm_scale * log2(e)
  float* part_acc;    // [B*H*nsplit, D] unnormalised partial outputs
  float* part_ml;     // [B*H*nsplit, 2] running max (log2 domain) and sum
  unsigned* merge_cnt;  // [units] split tickets (zero between calls), or null: separate combine
  int unit_spin;        // polls before the per-unit merge gives up (0: kUnitMergeSpin)
  int unit_never;       // test mode: the per-unit merge never sees its words (gives up)
  uint32_t* err;        // set to 1 when the per-unit merge gives up, or null
  // fused RoPE + new-token K/V write (ROPE kernels only)
  LLPartials qkv;          // [splits][B][(H + 2 KVH) * D] split-K partials (fp32, or int32 + scales)
  const void* qkv_bias;    // [(H + 2 KVH) * D] of the model dtype, or null
  const void* pos; int pos64;
  const float* cos_tab; const float* sin_tab; int64_t tab_stride;
  const int32_t* new_slots;  // [B] pool slot of each sequence's new token
  // optional quantisation of the output rows for the next int8 projection
  int8_t* qout; int64_t ldq; float* qscale; const float* qstatic;
};

// Partial kinds of the fused RoPE kernels (template MODE): 1 = fp32 partials
// from at most kRopeF32Splits splits, summed by one fixed, branch-free set of
// loads; 2 = any LLPartials (int32 with scales, or more fp32 splits). Kind 1
// exists so that its loads are not preceded by the conservative vmcnt(0) the
// compiler puts where the int32 and fp32 load sequences of a runtime branch
// share registers: that wait would drain the K/V copies issued just before
// and put a whole memory round trip in front of the q rebuild.
constexpr int kRopeF32Splits = 8;

// One job of the fused RoPE: 4 rotation pairs (i..i+3 with i+D/2..i+D/2+3) of
// the head whose columns start at hcol, with the arithmetic of the split-K
// RoPE/scatter kernel: sum of the partials in split order, + bias in fp32,
// rounded to T, rotated in fp32 with explicit FMAs, rounded to T. V heads are
// only rounded. Results go to LDS and, when glb is set, to global memory.
template <typename T, int D, int PK>
__device__ __forceinline__ void rope_job(const DecodeArgs& a, int64_t m, int64_t row, int hcol,
                                         int i, const float* cs, const float* sn, bool rotate,
                                         T* lds, T* glb) {
  constexpr int HALF = D / 2;
  const int c0 = hcol + i, c1 = c0 + HALF;
  // bias and the cos/sin entries first: their loads share the partials' round
  // trip. The bias is loaded unconditionally (from the partials, a valid
  // buffer wider than a row, when there is none) and selected after the sums:
  // a load used only under a branch is waited for inside it, one round trip
  // per element.
  const bool has_bias = a.qkv_bias != nullptr;
  const T* bsrc = has_bias ? (const T*)a.qkv_bias : (const T*)a.qkv.p;
  T rb0[4], rb1[4];
  float cv[4], sv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    rb0[e] = bsrc[c0 + e];
    rb1[e] = bsrc[c1 + e];
    cv[e] = cs[i + e];
    sv[e] = sn[i + e];
  }
  f32x4 x0, x1;
  if constexpr (PK == 1)
    ll_sum_splits4_pair_upto<kRopeF32Splits>((const float*)a.qkv.p, a.qkv.splits, a.qkv.sstride,
                                             row + c0, row + c1, x0, x1);
  else
    ll_partials_sum4_pair(a.qkv, row + c0, row + c1, m, c0, c1, x0, x1);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float s0 = x0[e] + ll_to_f32(rb0[e]), s1 = x1[e] + ll_to_f32(rb1[e]);
    x0[e] = has_bias ? s0 : x0[e];
    x1[e] = has_bias ? s1 : x1[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    T y0, y1;
    if (rotate) {
      const float u = ll_to_f32(ll_from_f32<T>(x0[e])), w = ll_to_f32(ll_from_f32<T>(x1[e]));
      ll_rope_pair(u, w, cv[e], sv[e], y0, y1);
    } else {
      y0 = ll_from_f32<T>(x0[e]);
      y1 = ll_from_f32<T>(x1[e]);
    }
    lds[i + e] = y0;
    lds[i + HALF + e] = y1;
    if (glb != nullptr) {
      glb[i + e] = y0;
      glb[i + HALF + e] = y1;
    }
  }
}

// Log-sum-exp merge of the partials of one (sequence, head) by one wave:
// lane l returns out[d = l + 64 q] (unrounded). Splits are taken SB at a time
// with all their loads issued before any is used (one memory round trip per
// SB splits).
template <int D, int SB>
__device__ __forceinline__ void combine_bh_sb(const DecodeArgs& a, int bh, int lane,
                                              float (&o)[D / 64]) {
  constexpr int DPL = D / 64;
  const int ns = a.nsplit;
  const int64_t p0 = (int64_t)bh * ns;  // partial rows of (b, h): p0 .. p0 + ns - 1
  float M = -INFINITY, L = 0.f, A[DPL];
#pragma unroll
  for (int q = 0; q < DPL; ++q) A[q] = 0.f;
  for (int s0 = 0; s0 < ns; s0 += SB) {
    // lane s < SB holds (m, l) of split s0 + s; rows past the last split are
    // clamped onto it and weighted 0
    float av[SB][DPL];
#pragma unroll
    for (int u = 0; u < SB; ++u)
#pragma unroll
      for (int q = 0; q < DPL; ++q)
        av[u][q] = a.part_acc[(p0 + min(s0 + u, ns - 1)) * D + lane + 64 * q];
    const int sl = min(s0 + (lane & (SB - 1)), ns - 1);
    const float m0 = a.part_ml[(p0 + sl) * 2];
    const float l = a.part_ml[(p0 + sl) * 2 + 1];
    // every load of this chunk is issued before the first use of any of them
    __builtin_amdgcn_sched_barrier(0);
    const float m = (lane < SB && s0 + lane < ns) ? m0 : -INFINITY;
    float mc = m;
#pragma unroll
    for (int off = SB / 2; off > 0; off >>= 1) mc = fmaxf(mc, __shfl_xor(mc, off, 64));
    mc = __shfl(mc, 0, 64);
    const float Mn = fmaxf(M, mc);
    if (Mn != -INFINITY) {
      const float r = exp2f(M - Mn);
      L *= r;
#pragma unroll
      for (int q = 0; q < DPL; ++q) A[q] *= r;
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const float w = exp2f(__shfl(m, u, 64) - Mn);  // 0 for splits past the last
        L += __shfl(l, u, 64) * w;
#pragma unroll
        for (int q = 0; q < DPL; ++q) A[q] += av[u][q] * w;
      }
    }
    M = Mn;
  }
#pragma unroll
  for (int q = 0; q < DPL; ++q) o[q] = L > 0.f ? A[q] / L : 0.f;
}

// SB = the split count rounded up to 4, 8 or 16 (rows past the last split
// weigh 0, so every SB gives the same sums)
template <int D>
__device__ __forceinline__ void combine_bh(const DecodeArgs& a, int bh, int lane, float (&o)[D / 64]) {
  if (a.nsplit <= 4) combine_bh_sb<D, 4>(a, bh, lane, o);
  else if (a.nsplit <= 8) combine_bh_sb<D, 8>(a, bh, lane, o);
  else combine_bh_sb<D, 16>(a, bh, lane, o);
}

// Split partials in the workspace: +0.0 is stored as -0.0 (the merges only
// add and multiply these words, where the two zeros give the same results),
// so that a zero word means "not written". Every merge zeroes the rows it
// consumed, so the partial rows are all zero between calls (the workspace
// starts zeroed), and the per-unit merge can poll the words themselves
// instead of waiting for their stores to be acknowledged.
__device__ __forceinline__ float part_word(float x) { return x == 0.f ? -0.f : x; }

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Zeroes the partial rows of (sequence, head) bh after one wave merged them
// (its loads have returned: their values were used).
template <int D>
__device__ __forceinline__ void clear_bh(const DecodeArgs& a, int bh, int lane) {
  const int64_t p0 = (int64_t)bh * a.nsplit;
  for (int s = 0; s < a.nsplit; ++s)
#pragma unroll
    for (int q = 0; q < D / 64; ++q) a.part_acc[(p0 + s) * D + lane + 64 * q] = 0.f;
  for (int i = lane; i < 2 * a.nsplit; i += 64) a.part_ml[p0 * 2 + i] = 0.f;
}

// XCD-aware mapping: the dispatcher deals the workgroups of a launch to the
// 8 XCDs round-robin, workgroup i to XCD (i + r) mod 8 for one r per launch
// (the round-robin continues from the previous launch, so r varies), and
// every workgroup of one sequence (all its KV heads and splits) is given an
// index of the same residue, so they all run on one XCD and share its L2.
__device__ __forceinline__ void map_block(int bid, int KVH, int nsplit, int& b, int& kvh,
                                          int& split) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per_seq = KVH * nsplit;
  const int k = slot / per_seq, r = slot - k * per_seq;
  b = k * 8 + xcd;
  kvh = r / nsplit;
  split = r - kvh * nsplit;
}

template <int D> struct TileGeom {
  static constexpr int ROWB = D * 2;            // bytes of one K or V row
  static constexpr int CH = ROWB / 16;          // 16 B chunks per row
  static constexpr int RPI = 64 / CH;           // rows per wave DMA instruction
  static constexpr int IPT = kTT / RPI;         // DMA instructions per tile, K or V
  static constexpr int TILE_B = 2 * kTT * ROWB; // K rows then V rows
  static constexpr int ROWS_PER_BANKS = 256 / ROWB;  // rows sharing one 256 B bank window
  static constexpr int RING_B = kWaves * kRing * TILE_B;
  static constexpr int CP = D + 4;  // floats per merge row (16 B aligned, staggers the banks)
  // a wave's merge rows (16 x CP accumulators, 16 maxima, 16 sums) sit in its
  // own tile ring, which is idle once the wave has left its token loop
  static constexpr int WAVE_B = kRing * TILE_B;
  static constexpr int MERGE_WAVE_B = 16 * CP * 4 + 2 * 16 * 4;
  static_assert(MERGE_WAVE_B <= WAVE_B, "merge rows must fit in a wave's ring");
  static constexpr int MAIN_B = RING_B;
  // LDS chunk position of global chunk c of tile row r (an involution)
  static __device__ __forceinline__ int swz(int c, int r) { return c ^ ((r / ROWS_PER_BANKS) & (CH - 1)); }
};

// Merge of a unit's splits by its split nsplit - 1, whose own partial
// (own_merge: the merge of its waves) stays in registers, one (head, 4 d)
// item per thread. That workgroup has the highest index of its unit, and
// workgroups start in index order on an XCD, so the NO = nsplit - 1 others it
// waits for started before it and wait for nothing themselves: they store
// their partial words as soon as they have them. A zero word is one not yet
// written. All splits of a unit run on one XCD (map_block), whose L2 the
// polls read; each poll issues every load before looking at any, and the
// first one is in flight while own_merge runs. The wait is bounded
// (a.unit_spin polls; the rows then come out NaN and *a.err, when given, is
// set to 1, as the decode step's fused launches report a wait that gave up).
// The merge is
// combine_bh's arithmetic, splits in order, so both merges give the same
// bits. The merged rows are zeroed for the next call.
template <typename T, int D, int NO, typename OwnMerge>
__device__ __forceinline__ void unit_merge_tail(const DecodeArgs& a, bool item, int b, int kvh,
                                                int g, int d0, int64_t pbase,
                                                const OwnMerge& own_merge) {
  const int ns = a.nsplit;
  const int no = ns - 1;
  const int64_t p0 = pbase + (int64_t)g * ns;  // this item's rows: p0 .. p0 + ns - 1
  float M, L;
  f32x4 A;
  if (item) {
    float am[NO][4], mm[NO], lm[NO];
    bool gave_up = false;
    uint32_t u[NO][6];
    auto poll = [&]() {
#pragma unroll
      for (int s = 0; s < NO; ++s) {
        const int64_t ps = p0 + min(s, no - 1);
        const uint32_t* wa = (const uint32_t*)(a.part_acc + ps * D + d0);
        const uint32_t* wm = (const uint32_t*)(a.part_ml + ps * 2);
#pragma unroll
        for (int q = 0; q < 4; ++q) u[s][q] = ld_agent(wa + q);
        u[s][4] = ld_agent(wm);
        u[s][5] = ld_agent(wm + 1);
      }
    };
    poll();
    own_merge(M, L, A);  // this workgroup's merge while the first poll is in flight
    for (int it = 0;; ++it) {
      bool ready = true;
#pragma unroll
      for (int s = 0; s < NO; ++s) {
#pragma unroll
        for (int q = 0; q < 4; ++q) am[s][q] = __uint_as_float(u[s][q]);
        mm[s] = __uint_as_float(u[s][4]);
        lm[s] = __uint_as_float(u[s][5]);
        const bool all = u[s][0] != 0u && u[s][1] != 0u && u[s][2] != 0u && u[s][3] != 0u &&
                         u[s][4] != 0u && u[s][5] != 0u;
        ready = ready && (s >= no || all);
      }
      if (ready && a.unit_never == 0) break;
      if (it >= a.unit_spin) {
        gave_up = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      poll();
    }
    float Mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < NO; ++s)
      if (s < no) Mx = fmaxf(Mx, mm[s]);
    Mx = fmaxf(Mx, M);
    float Lx = 0.f, Ax[4] = {0.f, 0.f, 0.f, 0.f};
    if (Mx != -INFINITY) {
#pragma unroll
      for (int s = 0; s < NO; ++s) {
        if (s < no) {
          const float w = exp2f(mm[s] - Mx);
          Lx += lm[s] * w;
#pragma unroll
          for (int q = 0; q < 4; ++q) Ax[q] += am[s][q] * w;
        }
      }
      const float w = exp2f(M - Mx);
      Lx += L * w;
#pragma unroll
      for (int q = 0; q < 4; ++q) Ax[q] += A[q] * w;
    }
    T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)(kvh * a.G + g) * a.o_sh + d0;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      op[q] = ll_from_f32<T>(gave_up ? __builtin_nanf("") : (Lx > 0.f ? Ax[q] / Lx : 0.f));
    if (gave_up && a.err != nullptr)
      __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int s = 0; s < no; ++s)
      *(f32x4*)&a.part_acc[(p0 + s) * D + d0] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  lds_barrier();  // every poll of the (m, l) words is done
  if (item && d0 == 0) {
    for (int i = 0; i < 2 * no; ++i) a.part_ml[p0 * 2 + i] = 0.f;
  }
}

// ROPE: q comes from the QKV projection's split-K partials (bias, RoPE) instead
// of a q tensor, and the workgroup whose split holds the sequence's last tile
// also builds the new token's K/V, patches the tile rows carrying that slot in
// its own LDS copy (its copies read the pool's old contents of the slot) and
// writes them to new_slots[b] in the pool on its way out. Precondition: a
// sequence's new slot appears in no other sequence's first seq_len entries
// and in its own only within the last split (the decode step puts it at
// seq_len - 1).
// The split stage, for both kernels below. p_len .. idx64 are the fields of
// the first loads (lengths, request rows, positions, new slots, the grid
// geometry); idx64: bit 0 lengths, bit 1 request rows, bit 2 positions are
// int64.
template <typename T, int D, int MODE>
__device__ __forceinline__ void decode_attn_split_stage(
    const int32_t* __restrict__ p_len, const int32_t* __restrict__ p_rid,
    const int32_t* __restrict__ p_pos, const int32_t* __restrict__ p_nslot, int KVH, int nsplit,
    int B, int idx64, const DecodeArgs& a) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec4<T>::type V4;
  typedef TileGeom<D> TG;
  constexpr bool ROPE = MODE != 0;  // q from the QKV partials (1: fp32, 2: any kind)
  constexpr int DS = D / 32;  // k-steps of the S^T product
  constexpr int DB = D / 16;  // 16-wide d blocks of the output
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int32_t* s_slots = (int32_t*)(smem + TG::MAIN_B);

  int b, kvh, split;
  map_block(blockIdx.x, KVH, nsplit, b, kvh, split);
  if (b >= B) return;
  const int unit = b * KVH + kvh;
  // sequence length and request row (and with ROPE the position and the new
  // slot), all loads in flight together and before anything that reads the
  // argument block (the low word of an int64 entry is the value: lengths,
  // rows and positions are below 2^31)
  const int32_t len32 = p_len[(idx64 & 1) ? 2 * b : b];
  const int32_t rid32 = p_rid[(idx64 & 2) ? 2 * b : b];
  int32_t pos32 = 0, new_slot = 0;
  if constexpr (MODE != 0) {
    pos32 = p_pos[(idx64 & 4) ? 2 * b : b];
    new_slot = p_nslot[b];
  }
  // the wave index as a scalar (threadIdx.x / 64 is the same in every lane
  // of a wave): branches on it are scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;  // MFMA column (query head within the group) / row
  const int j = lane >> 4;  // lane group

  // Q^T as the B operand: column n = head kvh*G + n, k-slots = d 32*s + 8*j + 0..7.
  // Loaded first (it does not depend on the lengths); columns n >= G read
  // head G - 1.
  V8 qb[DS];
  T* s_q = (T*)(smem + TG::MAIN_B + (size_t)a.slots_cap * 4);  // ROPE: [G][D] rotated q
  T* s_kv = s_q + a.G * D;                                     // ROPE: new token's K, V
  constexpr int QD = D / 8;  // RoPE jobs per head
  if constexpr (!ROPE) {
    const int hq = kvh * a.G + min(n, a.G - 1);
    const T* qp = (const T*)a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh;
#pragma unroll
    for (int s = 0; s < DS; ++s) qb[s] = *(const V8*)(qp + 32 * s + 8 * j);
  }
  // The RoPE jobs come after the first slot loads are issued, so that the
  // two dependent chains (length/row -> slots, position -> cos/sin) overlap.
  asm volatile("" ::"s"(len32), "s"(rid32), "s"(pos32), "s"(new_slot));  // the loads are in
  int64_t len = len32 > a.max_len ? a.max_len : len32;
  const int64_t rid = rid32;
  const int32_t* slot_row = a.r2t + rid * a.r2t_s;
  const int ntiles = (int)((len + kTT - 1) / kTT);
  const int per = (ntiles + nsplit - 1) / nsplit;
  const int tb = min(ntiles, split * per);
  const int te = min(ntiles, tb + per);
  const int64_t tok0 = (int64_t)tb * kTT;
  const int ntok = (int)(min(len, (int64_t)te * kTT) - tok0);  // tokens of this split (may be 0)

  const char* kbase = (const char*)((const T*)a.k + (int64_t)kvh * a.k_sh);
  const char* vbase = (const char*)((const T*)a.v + (int64_t)kvh * a.v_sh);
  const int64_t kst = a.k_st * (int64_t)sizeof(T), vst = a.v_st * (int64_t)sizeof(T);
  char* ring = smem + wave * kRing * TG::TILE_B;
  const int nw = (te - tb - wave + kWaves - 1) / kWaves;  // tiles of this wave (may be <= 0)

  // slot ids of this wave's tiles (wave, wave + kWaves, ... of the split) ->
  // LDS, up to 16 tiles per round with every load of a round in flight
  // together; tail entries point at slot 0 (masked later). Only this wave reads them
  // (K/V copy addresses, the writer's patch test), and a wave's LDS accesses
  // are ordered, so no barrier stands between the slot loads and the wave's
  // first K/V copies. The first round's loads are always issued (every
  // index is clamped to a valid entry), so that the RoPE jobs' loads below
  // share their round trip.
  auto load_round = [&](int r0, int32_t (&sl)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = (wave + kWaves * (4 * (r0 + u) + (lane >> 4))) * kTT + (lane & 15);
      const int64_t t = min(tok0 + i, len > 0 ? len - 1 : (int64_t)0);  // always a valid entry
      sl[u] = slot_row[t];
    }
  };
  auto store_round = [&](int r0, const int32_t (&sl)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tw = wave + kWaves * (4 * (r0 + u) + (lane >> 4));  // tile within the split
      const int i = tw * kTT + (lane & 15);                         // token within the split
      if (tw < te - tb) s_slots[i] = (i < ntok) ? sl[u] : 0;
    }
  };
  int32_t sl0[4];
  load_round(0, sl0);

  // ROPE: q of the group's heads into LDS; the split holding the last tile
  // (split 0 for an empty sequence) also writes the new token's K and V (the
  // last 2 * QD threads, one job each). Their loads are issued before any
  // K/V copy: waiting for them then waits for no copy (loads and copies
  // share the in-order vmcnt counter).
  bool writer = false;
  int jb = -1;  // ROPE, writer workgroup: this thread's new K/V job, or < 0
  if constexpr (ROPE) {
    const int64_t qkv_row = (int64_t)b * ((a.H + 2 * a.KVH) * D);
    const float* cs = a.cos_tab + (int64_t)pos32 * a.tab_stride;
    const float* sn = a.sin_tab + (int64_t)pos32 * a.tab_stride;
    if ((int)threadIdx.x < a.G * QD) {  // G * QD <= 16 * D / 8 <= 256
      const int g = threadIdx.x / QD, i = (threadIdx.x % QD) * 4;
      rope_job<T, D, MODE>(a, b, qkv_row, (kvh * a.G + g) * D, i, cs, sn, true, s_q + g * D,
                     nullptr);
    }
    writer = split == (ntiles > 0 ? (ntiles - 1) / per : 0);
    jb = (int)threadIdx.x - (kWaves * 64 - 2 * QD);
    if (writer && jb >= 0) {
      const bool isv = jb >= QD;
      const int i = (isv ? jb - QD : jb) * 4;
      rope_job<T, D, MODE>(a, b, qkv_row, (a.H + (isv ? a.KVH : 0) + kvh) * D, i, cs, sn,
                     !isv, s_kv + (isv ? D : 0), nullptr);
    }
  }
  // The new token's K/V go to the pool from s_kv when the workgroup leaves
  // (no split reads that slot from the pool in this launch; the writer's own
  // tile copy is patched from s_kv). Stored here, they would sit in the
  // vector memory counter ahead of the K/V copies, and the first copy would
  // wait for their acknowledgement.
  auto store_new_kv = [&]() {
    if constexpr (ROPE) {
      if (writer && jb >= 0) {
        const bool isv = jb >= QD;
        const int i = (isv ? jb - QD : jb) * 4;
        T* glb = isv ? (T*)a.v + (int64_t)new_slot * a.v_st + (int64_t)kvh * a.v_sh
                     : (T*)a.k + (int64_t)new_slot * a.k_st + (int64_t)kvh * a.k_sh;
        const T* src = s_kv + (isv ? D : 0);
        *(uint64_t*)(glb + i) = *(const uint64_t*)(src + i);
        *(uint64_t*)(glb + i + D / 2) = *(const uint64_t*)(src + i + D / 2);
      }
    }
  };
  store_round(0, sl0);
  for (int r0 = 4; 4 * r0 < nw; r0 += 4) {  // further rounds of 16 tiles (long splits)
    int32_t sl[4];
    load_round(r0, sl);
    store_round(r0, sl);
  }

  // DMA lane geometry: lane -> (row within an instruction's rows, LDS chunk position)
  const int dr = lane / TG::CH, dp = lane % TG::CH;
  auto issue = [&](int k) {
    const int t0 = (wave + k * kWaves) * kTT;  // token offset of the tile within the split
    char* buf = ring + (k % kRing) * TG::TILE_B;
#pragma unroll
    for (int i = 0; i < TG::IPT; ++i) {
      const int r = i * TG::RPI + dr;
      const int64_t slot = s_slots[t0 + r];
      const int c = TG::swz(dp, r);
      dma16(kbase + slot * kst + c * 16, buf + i * 1024);
      dma16(vbase + slot * vst + c * 16, buf + kTT * TG::ROWB + i * 1024);
    }
  };
  // The first tile's copies go out before the q barrier; the next tile's at
  // the top of the token loop. (Issuing both here, or refilling a buffer
  // after computing it, measured no faster: the LDS read of the second
  // tile's slot ids after the first tile's copies makes the compiler wait
  // for those copies, as it cannot tell the LDS buffers apart.)
  static_assert(kRing == 2, "the tile waits below assume two buffers per wave");
  if (0 < nw) issue(0);

  if constexpr (ROPE) {
    lds_barrier();  // s_q and s_kv are complete (the copies stay in flight)
    const T* qs = s_q + min(n, a.G - 1) * D;
#pragma unroll
    for (int s = 0; s < DS; ++s) qb[s] = *(const V8*)(qs + 32 * s + 8 * j);
  }
  // (columns n >= G hold a copy of head G - 1: their scores and sums are
  // finite and their outputs are never stored)

  f32x4 acc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max of head n (log2 domain)
  float l_run = 0.f;        // this lane's share of the running sum

  // ---- per-tile pieces of the token loop
  // ROPE: rows of a tile that carry the new slot get the fresh K/V (in-wave
  // LDS order puts these writes before the reads that follow)
  auto patch = [&](char* kb, int t0) {
    if constexpr (ROPE) {
      if (writer) {
        const bool hit = (t0 + n) < ntok && s_slots[t0 + n] == new_slot;
        uint64_t hits = __ballot(hit) & 0xffffull;
        while (hits) {
          const int r = __builtin_ctzll(hits);
          hits &= hits - 1;
          if (lane < 2 * TG::CH) {
            const int isv = lane >= TG::CH ? 1 : 0;
            const int cc = lane - isv * TG::CH;
            const u32x4 v = *(const u32x4*)((const char*)s_kv + isv * TG::ROWB + cc * 16);
            *(u32x4*)(kb + isv * kTT * TG::ROWB + r * TG::ROWB + TG::swz(cc, r) * 16) = v;
          }
        }
      }
    }
  };
  // S^T block of a tile: rows = tokens 4j+i, column = head n; scaled into
  // the log2 domain, -inf past the split's end
  auto scores = [&](const char* kb, int t0, bool (&ok)[4], float (&x)[4]) {
    f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const V8 ka = *(const V8*)(kb + n * TG::ROWB + TG::swz(4 * s + j, n) * 16);
      s4 = mfma16x16x32(ka, qb[s], s4);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ok[i] = (t0 + 4 * j + i) < ntok;
      x[i] = ok[i] ? s4[i] * a.scale_log2 : -INFINITY;
    }
  };
  // P stays (nearly) fp32 as in the reference's fp32 p * v accumulation
  // (flash_decoding.py:94-98): p = hi + lo with both parts in T, two MFMAs,
  // relative error of hi + lo about 2^-17 (bf16) / 2^-22 (fp16). Returns the
  // sum of the tile's p.
  auto probs = [&](const float (&x)[4], float m_new, V4& pb, V4& pl) {
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = exp2f(x[i] - m_new);
      psum += p;
      const T ph = (T)p;
      pb[i] = bits16(ph);
      pl[i] = bits16((T)(p - ll_to_f32(ph)));
    }
    return psum;
  };
  // O^T[d, head] += V^T[d, tok] . P^T[tok, head]; k-slot i of lane group j
  // is token 4j+i. The V^T fragment (d = 16c + n, tokens 4j..4j+3) comes
  // from one transposing LDS read per d block: local lane 4e + q of lane
  // group j addresses row 4j + e, columns 16c + 4q .. 16c + 4q + 3, so
  // lane n receives V[4j + e][16c + n] as its element e.
  const int vrow = 4 * j + (n >> 2);
  auto v_read = [&](const char* vb, int c) {
    const int chunk = 2 * c + ((n & 3) >> 1);  // 16-byte chunk of columns 16c + 4q
    return ll_lds_read_tr16(vb + vrow * TG::ROWB + TG::swz(chunk, vrow) * 16 + (n & 1) * 8);
  };
  auto v_frag = [&](s16x4 raw, const bool (&ok)[4]) {
    V4 va = as_v4(raw, V4{});
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (!ok[i]) va[i] = bits16((T)0.f);  // tokens past the split's end
    return va;
  };
  auto row_max = [&](float t) {  // max over the 4 lane groups (all 16 tokens of a column)
    t = fmaxf(t, __shfl_xor(t, 16, 64));
    return fmaxf(t, __shfl_xor(t, 32, 64));
  };

  for (int k = 0; k < nw; ++k) {
    if (k + 1 < nw) {
      issue(k + 1);
      vm_wait<2 * TG::IPT>();  // tile k's copies are done, tile k + 1's in flight
    } else {
      vm_wait<0>();
    }
    char* kb = ring + (k % kRing) * TG::TILE_B;
    const char* vb = kb + kTT * TG::ROWB;
    const int t0 = (wave + k * kWaves) * kTT;
    patch(kb, t0);
    bool ok[4];
    float x[4];
    scores(kb, t0, ok, x);
    const float tmax = row_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
    const float m_new = fmaxf(m_run, tmax);  // finite: the tile's first token is valid
    const float alpha = exp2f(m_run - m_new);
    V4 pb, pl;
    const float psum = probs(x, m_new, pb, pl);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    s16x4 vr[DB];
#pragma unroll
    for (int c = 0; c < DB; ++c) vr[c] = v_read(vb, c);
    ll_lds_wait_tie(vr);
#pragma unroll
    for (int c = 0; c < DB; ++c) {
      const V4 va = v_frag(vr[c], ok);
      acc[c] = mfma16x16x16(va, pl, mfma16x16x16(va, pb, acc[c] * alpha));
    }
    // this buffer is refilled by the next issue: its LDS reads must be done
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // total sum of head n across the 4 lane groups
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  // ---- merge the waves of this workgroup. Each wave writes its rows into its
  // own ring (its DMAs have landed and its LDS reads are done), so only the
  // barrier after the writes is needed.
  auto comb_acc = [&](int w, int g) { return (float*)(smem + w * TG::WAVE_B) + g * TG::CP; };
  auto comb_m = [&](int w) { return (float*)(smem + w * TG::WAVE_B + 16 * TG::CP * 4); };
  auto comb_l = [&](int w) { return (float*)(smem + w * TG::WAVE_B + 16 * TG::CP * 4 + 64); };
  const int G = a.G;
  // acc[c][i] holds O^T[d = 16c + 4j + i][head n]; only the G real heads are kept
  if (n < G) {
#pragma unroll
    for (int c = 0; c < DB; ++c) *(f32x4*)(comb_acc(wave, n) + 16 * c + 4 * j) = acc[c];
    if (j == 0) {
      comb_m(wave)[n] = m_run;
      comb_l(wave)[n] = l_run;
    }
  }
  __syncthreads();

  // Per-unit merge (several splits, rows not quantised): split nsplit - 1 of
  // every (sequence, KV head) merges the others' partials (unit_merge_tail).
  const bool whole_row = a.qout != nullptr;
  const bool unit_merge = a.merge_cnt != nullptr && !whole_row && a.nsplit <= kUnitMergeSplits;

  // four consecutive d of one head per thread (G * D / 4 <= kWaves * 64)
  constexpr int DQ = D / 4;
  const int64_t pbase = ((int64_t)b * a.H + (int64_t)kvh * G) * a.nsplit;
  const int e = threadIdx.x;
  const bool item = e < G * DQ;
  const int g = item ? e / DQ : 0, d0 = item ? (e - g * DQ) * 4 : 0;
  // this workgroup's (max, sum, accumulators) of the thread's item
  auto wave_merge = [&](float& M, float& L, f32x4& A) {
    M = -INFINITY;
    L = 0.f;
    A = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (item) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, comb_m(w)[g]);
      if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const float sc = exp2f(comb_m(w)[g] - M);
          L += comb_l(w)[g] * sc;
          const f32x4 v = *(const f32x4*)(comb_acc(w, g) + d0);
#pragma unroll
          for (int i = 0; i < 4; ++i) A[i] += v[i] * sc;
        }
      }
    }
  };
  if (unit_merge && split == a.nsplit - 1) {
    if (a.nsplit == 2)
      unit_merge_tail<T, D, 1>(a, item, b, kvh, g, d0, pbase, wave_merge);
    else if (a.nsplit == 3)
      unit_merge_tail<T, D, 2>(a, item, b, kvh, g, d0, pbase, wave_merge);
    else if (a.nsplit == 4)
      unit_merge_tail<T, D, 3>(a, item, b, kvh, g, d0, pbase, wave_merge);
    else
      unit_merge_tail<T, D, kUnitMergeSplits - 1>(a, item, b, kvh, g, d0, pbase, wave_merge);
    store_new_kv();
    return;
  }
  float M, L;
  f32x4 A;
  wave_merge(M, L, A);
  if (a.nsplit == 1) {
    if (item) {
      T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)(kvh * G + g) * a.o_sh + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) op[i] = ll_from_f32<T>(L > 0.f ? A[i] / L : 0.f);
    }
    store_new_kv();
    return;
  }
  if (item) {
    const int64_t p = pbase + (int64_t)g * a.nsplit + split;
    *(f32x4*)&a.part_acc[p * D + d0] = (f32x4){part_word(A[0]), part_word(A[1]),
                                               part_word(A[2]), part_word(A[3])};
    if (d0 == 0) {
      a.part_ml[p * 2] = part_word(M);
      a.part_ml[p * 2 + 1] = part_word(L);
    }
  }
  store_new_kv();
  if (a.merge_cnt == nullptr) return;

  if (unit_merge) return;

  __shared__ unsigned s_ticket;
  // ---- more splits than the per-unit merge holds, or quantised rows: the
  // last split of the unit (or, with quantised rows, the last workgroup of the
  // sequence, which merges all its heads and quantises the row) merges after
  // every partial store has been acknowledged by the XCD's L2 (the vector L1
  // is write-through) and drops its own L1 lines before reading them.
  const unsigned last = (unsigned)((whole_row ? a.KVH : 1) * a.nsplit - 1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    s_ticket = __builtin_amdgcn_atomic_inc32(a.merge_cnt + (whole_row ? b : unit), last,
                                             __ATOMIC_RELAXED, "agent");
  __syncthreads();
  if (s_ticket != last) return;
  asm volatile("buffer_inv sc0" ::: "memory");
  if (!whole_row) {
    for (int gg = wave; gg < G; gg += kWaves) {
      float o[D / 64];
      const int bh = b * a.H + kvh * G + gg;
      combine_bh<D>(a, bh, lane, o);
      clear_bh<D>(a, bh, lane);
      T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)(kvh * G + gg) * a.o_sh;
#pragma unroll
      for (int q = 0; q < D / 64; ++q) op[lane + 64 * q] = ll_from_f32<T>(o[q]);
    }
    return;
  }
  // the stored row is kept in LDS (the tile rings are idle) for the codes:
  // by ll_quant_per_token's rule, or with the calibrated scale *a.qstatic
  float* row = (float*)smem;
  __shared__ float s_red[kWaves];
  float amax = 0.f;
  for (int h = wave; h < a.H; h += kWaves) {
    float o[D / 64];
    combine_bh<D>(a, b * a.H + h, lane, o);
    clear_bh<D>(a, b * a.H + h, lane);
    T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
#pragma unroll
    for (int q = 0; q < D / 64; ++q) {
      const T v = ll_from_f32<T>(o[q]);
      op[lane + 64 * q] = v;
      const float y = ll_to_f32(v);
      row[h * D + lane + 64 * q] = y;
      amax = fmaxf(amax, fabsf(y));
    }
  }
  amax = ll_wave_max(amax);
  if (lane == 0) s_red[wave] = amax;
  __syncthreads();
  float sc;
  if (a.qstatic != nullptr) {
    sc = *a.qstatic;
  } else {
    float mx = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, s_red[w]);
    sc = mx / 127.f;
    if (!(sc > 0.f)) sc = 1.f;
  }
  if (threadIdx.x == 0) a.qscale[b] = sc;
  int8_t* qrow = a.qout + (int64_t)b * a.ldq;
  for (int i = threadIdx.x; i < a.H * D; i += kWaves * 64) qrow[i] = ll_quant1(row[i], sc);
}

// Plain attention (q given): the fields of the first loads come as scalar
// arguments ahead of the DecodeArgs block. gfx950 preloads leading scalar
// kernel arguments into SGPRs at dispatch, so the length and request-row
// loads do not wait for the argument block's load (config 2: 10.35 -> 9.95
// us per op).
template <typename T, int D>
__global__ __launch_bounds__(kWaves * 64) void decode_attn_dma_kernel(
    const int32_t* __restrict__ p_len, const int32_t* __restrict__ p_rid, int KVH, int nsplit,
    int B, int idx64, DecodeArgs a) {
  decode_attn_split_stage<T, D, 0>(p_len, p_rid, nullptr, nullptr, KVH, nsplit, B, idx64, a);
}

// Fused RoPE variants: the argument block only (their q rebuild waits for the
// positions' round trip either way, and preloaded arguments made the W8A8
// decode step 7 us slower).
template <typename T, int D, int MODE>
__global__ __launch_bounds__(kWaves * 64) void decode_attn_rope_kernel(DecodeArgs a) {
  asm volatile("" ::"s"(a.seq_len), "s"(a.req_idx), "s"(a.len64), "s"(a.req64), "s"(a.pos),
               "s"(a.pos64), "s"(a.new_slots));  // the four data loads go out together
  const int idx64 = (a.len64 ? 1 : 0) | (a.req64 ? 2 : 0) | (a.pos64 ? 4 : 0);
  decode_attn_split_stage<T, D, MODE>((const int32_t*)a.seq_len, (const int32_t*)a.req_idx,
                                      (const int32_t*)a.pos, a.new_slots, a.KVH, a.nsplit, a.B,
                                      idx64, a);
}

// Separate merge kernels, for the shapes the split stage cannot merge itself
// (more than kMergeUnits units, or a quantised row larger than the tile
// rings): one wave per (sequence, head).
template <typename T, int D>
__global__ __launch_bounds__(kCombWaves * 64) void decode_attn_combine_kernel(DecodeArgs a) {
  constexpr int DPL = D / 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int bh = blockIdx.x * kCombWaves + wave;
  if (bh >= a.B * a.H) return;
  const int b = bh / a.H, h = bh - b * a.H;
  float o[DPL];
  combine_bh<D>(a, bh, lane, o);
  clear_bh<D>(a, bh, lane);
  T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
#pragma unroll
  for (int q = 0; q < DPL; ++q) op[lane + 64 * q] = ll_from_f32<T>(o[q]);
}

// Combine of one sequence per workgroup (HPW heads per wave, H <= 16 * HPW),
// then the o_proj input quantisation of the stored row out[b] (H * D values):
// codes by ll_quant_per_token's rule, or by *a.qstatic when set.
template <typename T, int D, int HPW>
__global__ __launch_bounds__(1024) void decode_attn_combine_quant_kernel(DecodeArgs a) {
  constexpr int DPL = D / 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int nw = blockDim.x >> 6;
  const int b = blockIdx.x;
  float y[HPW][DPL];
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int h = wave + k * nw;
    if (h < a.H) {
      float o[DPL];
      combine_bh<D>(a, b * a.H + h, lane, o);
      clear_bh<D>(a, b * a.H + h, lane);
      T* op = (T*)a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
#pragma unroll
      for (int q = 0; q < DPL; ++q) {
        const T v = ll_from_f32<T>(o[q]);
        op[lane + 64 * q] = v;
        y[k][q] = ll_to_f32(v);
        amax = fmaxf(amax, fabsf(y[k][q]));
      }
    }
  }
  float s;
  if (a.qstatic != nullptr) {
    s = *a.qstatic;
  } else {
    __shared__ float red[16];
    amax = ll_wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    float mx = 0.f;
    for (int w = 0; w < nw; ++w) mx = fmaxf(mx, red[w]);
    s = mx / 127.f;
    if (!(s > 0.f)) s = 1.f;
  }
  if (threadIdx.x == 0) a.qscale[b] = s;
  int8_t* qrow = a.qout + (int64_t)b * a.ldq;
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int h = wave + k * nw;
    if (h < a.H) {
#pragma unroll
      for (int q = 0; q < DPL; ++q) qrow[h * D + lane + 64 * q] = ll_quant1(y[k][q], s);
    }
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
  int64_t len = ll_load_idx(a.seq_len, b, a.len64);
  if (len > a.max_len) len = a.max_len;
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

constexpr int kMaxSplitTokens = 4096;  // LDS slot table bound per split (16 KB)
constexpr int kSplitCostTiles2 = 13;    // twice the cost of one more split, in 16-token tiles
constexpr int kMaxSplitsFill = 16;      // split bound from 8 units up (head_dim 128)

int choose_nsplit(int B, int KVH, int64_t max_len, int64_t head_dim) {
  const int units = B * KVH;
  const int64_t tiles = (max_len + kTT - 1) / kTT;
  // At most one dispatch round of the 256 CUs (as many split-stage
  // workgroups per CU as their LDS allows: one at head_dim 128, two at 64),
  // every wave at least one tile, the slot table bounded.
  // Measured at 40 sequences x 2 KV heads: one workgroup of 8 waves per CU
  // beats two of 4 waves from 600 tokens up (fewer splits to merge, the same
  // bytes in flight per CU).
  const int64_t main_b = head_dim == 64 ? TileGeom<64>::MAIN_B : TileGeom<128>::MAIN_B;
  const int per_cu = (int)(160 * 1024 / (main_b + 8192)) > 1 ? (int)(160 * 1024 / (main_b + 8192)) : 1;
  int ns = 256 * per_cu / units;
  const int64_t max_ns = tiles / kWaves;
  if (ns > max_ns) ns = (int)max_ns;
  const int64_t min_ns = (tiles * kTT + kMaxSplitTokens - 1) / kMaxSplitTokens;
  if (ns < min_ns) ns = (int)min_ns;
  if (ns < 1) ns = 1;
  // head_dim 128, from a sweep of split counts (16 or 12 query heads per 2
  // KV heads, 4-64 sequences, 300-8000 tokens):
  // * at most 16 splits from 8 units up: the merging workgroup reads every
  //   split's partial rows (4 x 8000 tokens: 32 splits 27.2 us, 16 16.1);
  // * from 64 units up (one dispatch round holds at most 4 splits), the
  //   count with the least (tiles of a split) + kSplitCostTiles2 / 2 per
  //   split: one split more costs about 6.5 tile times there, a workgroup's
  //   ramp and a longer merge (40 x 600 tokens: 2 splits 10.34 us, 3 10.64;
  //   40 x 700: 2 splits 11.54, 3 11.26; 32 x 600: 2 splits 10.02, 4 10.28).
  //   With fewer units the CUs left idle by fewer splits cost more than the
  //   merge, and the count above stands.
  if (head_dim == 128) {
    if (units >= 8 && ns > kMaxSplitsFill) ns = min_ns > kMaxSplitsFill ? (int)min_ns : kMaxSplitsFill;
    if (units >= 64) {
      int64_t best = -1;
      const int lo = min_ns > 1 ? (int)min_ns : 1;
      for (int s = lo, hi = ns; s <= hi; ++s) {
        const int64_t c = 2 * ((tiles + s - 1) / s) + kSplitCostTiles2 * s;
        if (best < 0 || c < best) {
          best = c;
          ns = s;
        }
      }
    }
  }
  return ns;
}

int64_t align256(int64_t x) { return ((x + 255) / 256) * 256; }



template <int D, int MODE>
void launch_split_stage(const DecodeArgs& a, int dtype, unsigned grid, size_t lds,
                        hipStream_t stream) {
  const int idx64 = (a.len64 ? 1 : 0) | (a.req64 ? 2 : 0) | (a.pos64 ? 4 : 0);
  const int32_t* p_len = (const int32_t*)a.seq_len;
  const int32_t* p_rid = (const int32_t*)a.req_idx;
  if constexpr (MODE == 0) {
    if (dtype == LL_BF16)
      hipLaunchKernelGGL((decode_attn_dma_kernel<__bf16, D>), dim3(grid), dim3(kWaves * 64), lds,
                         stream, p_len, p_rid, a.KVH, a.nsplit, a.B, idx64, a);
    else
      hipLaunchKernelGGL((decode_attn_dma_kernel<_Float16, D>), dim3(grid), dim3(kWaves * 64), lds,
                         stream, p_len, p_rid, a.KVH, a.nsplit, a.B, idx64, a);
  } else {
    if (dtype == LL_BF16)
      hipLaunchKernelGGL((decode_attn_rope_kernel<__bf16, D, MODE>), dim3(grid),
                         dim3(kWaves * 64), lds, stream, a);
    else
      hipLaunchKernelGGL((decode_attn_rope_kernel<_Float16, D, MODE>), dim3(grid),
                         dim3(kWaves * 64), lds, stream, a);
  }
}

template <int D>
void launch_combine(const DecodeArgs& a, int dtype, hipStream_t stream) {
  if (a.qout != nullptr) {
    const int nw = a.H < 16 ? a.H : 16;
    const dim3 qgrid((unsigned)a.B), qblock((unsigned)(64 * nw));
    const bool two = a.H > 16;
    if (dtype == LL_BF16) {
      if (two) hipLaunchKernelGGL((decode_attn_combine_quant_kernel<__bf16, D, 2>), qgrid, qblock, 0, stream, a);
      else hipLaunchKernelGGL((decode_attn_combine_quant_kernel<__bf16, D, 1>), qgrid, qblock, 0, stream, a);
    } else {
      if (two) hipLaunchKernelGGL((decode_attn_combine_quant_kernel<_Float16, D, 2>), qgrid, qblock, 0, stream, a);
      else hipLaunchKernelGGL((decode_attn_combine_quant_kernel<_Float16, D, 1>), qgrid, qblock, 0, stream, a);
    }
    return;
  }
  const dim3 cgrid((unsigned)((a.B * a.H + kCombWaves - 1) / kCombWaves));
  if (dtype == LL_BF16)
    hipLaunchKernelGGL((decode_attn_combine_kernel<__bf16, D>), cgrid, dim3(kCombWaves * 64), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((decode_attn_combine_kernel<_Float16, D>), cgrid, dim3(kCombWaves * 64), 0,
                       stream, a);
}

// Workspace layout when the sequences are split: [kMergeUnits split tickets]
// [partial acc][partial (m, l)]. The tickets sit at a fixed offset so that
// calls of every shape sharing one workspace find them at zero.
constexpr int kMergeUnits = 4096;
constexpr int64_t kTicketBytes = kMergeUnits * 4;

// Whether the split stage may merge its splits itself (it needs every
// workgroup of a sequence on one XCD, which the dispatcher's round-robin
// gives; ll_decode_attention_xcc_probe checks it). Off: the separate merge
// kernels, which need no such premise.
std::atomic<int> g_same_launch_merge{1};

int64_t workspace_bytes_for(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t max_len) {
  const int ns = choose_nsplit((int)batch, (int)kv_heads, max_len, head_dim);
  if (ns <= 1) return 0;
  const int64_t parts = batch * q_heads * ns;
  return kTicketBytes                      // split tickets
         + align256(parts * head_dim * 4)  // partial acc
         + align256(parts * 2 * 4);        // partial (m, l)
}

// Split stage of the MFMA path (which merges the splits itself, or is followed
// by a separate merge kernel past kMergeUnits units); a has
// every field but the split geometry and the workspace pointers set.
int launch_mfma(DecodeArgs& a, int64_t head_dim, int dtype, bool rope, int64_t max_len,
                void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  a.nsplit = choose_nsplit(a.B, a.KVH, max_len, head_dim);
  if (a.unit_spin <= 0) a.unit_spin = kUnitMergeSpin;
  if (a.nsplit > 1) {
    const int64_t need = workspace_bytes_for(a.B, a.H, a.KVH, head_dim, max_len);
    LL_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                 "decode attention: workspace too small (need %lld bytes, got %lld)",
                 (long long)need, (long long)workspace_bytes);
    char* w = (char*)workspace;
    // merge in the split stage: per (sequence, KV head), or per sequence when
    // the rows are quantised (the row must fit in the tile rings' LDS)
    const int64_t row_b = (int64_t)a.H * head_dim * 4;
    const bool fits = a.qout == nullptr
                          ? a.units <= kMergeUnits
                          : (a.B <= kMergeUnits &&
                             row_b <= (head_dim == 128 ? TileGeom<128>::MAIN_B
                                                       : TileGeom<64>::MAIN_B));
    a.merge_cnt = (fits && g_same_launch_merge.load(std::memory_order_relaxed)) ? (unsigned*)w
                                                                                 : nullptr;
    w += kTicketBytes;
    const int64_t parts = (int64_t)a.B * a.H * a.nsplit;
    a.part_acc = (float*)w;
    w += align256(parts * head_dim * 4);
    a.part_ml = (float*)w;
  }
  const int64_t tiles = (max_len + kTT - 1) / kTT;
  a.slots_cap = (int)((tiles + a.nsplit - 1) / a.nsplit) * kTT;
  const int groups = (a.B + 7) / 8;  // sequences per XCD
  const unsigned grid = (unsigned)(groups * 8 * a.KVH * a.nsplit);
  const size_t extra = (size_t)a.slots_cap * 4 + (rope ? (size_t)(a.G + 2) * head_dim * 2 : 0);
  const int mode = !rope ? 0 : (!a.qkv.i32 && a.qkv.splits <= kRopeF32Splits) ? 1 : 2;
  if (head_dim == 128) {
    const size_t lds = TileGeom<128>::MAIN_B + extra;
    if (mode == 1) launch_split_stage<128, 1>(a, dtype, grid, lds, stream);
    else if (mode == 2) launch_split_stage<128, 2>(a, dtype, grid, lds, stream);
    else launch_split_stage<128, 0>(a, dtype, grid, lds, stream);
  } else {
    const size_t lds = TileGeom<64>::MAIN_B + extra;
    if (mode == 1) launch_split_stage<64, 1>(a, dtype, grid, lds, stream);
    else if (mode == 2) launch_split_stage<64, 2>(a, dtype, grid, lds, stream);
    else launch_split_stage<64, 0>(a, dtype, grid, lds, stream);
  }
  if (a.nsplit > 1) {
    if (a.merge_cnt == nullptr) {
      if (head_dim == 128) launch_combine<128>(a, dtype, stream);
      else launch_combine<64>(a, dtype, stream);
    }
  } else if (a.qout != nullptr) {
    // one split: the split stage stored the rows; quantise them here
    const int64_t W = (int64_t)a.H * head_dim;
    const int rc = a.qstatic != nullptr
                       ? ll_quant_static(a.out, a.o_sb, a.B, W, dtype, a.qstatic, a.qout, a.ldq,
                                         a.qscale, stream)
                       : ll_quant_per_token(a.out, a.o_sb, a.B, W, dtype, a.qout, a.ldq, a.qscale,
                                            stream);
    if (rc != LL_OK) return rc;
  }
  LL_RETURN_LAUNCH();
}

// The XCD (hardware register XCC_ID) each workgroup runs on, for the premise
// of the same-launch split merge: workgroup i of a grid runs on XCD
// (i + r) mod 8 with one r for the whole launch.
__global__ void xcc_probe_kernel(int32_t* __restrict__ out, int n) {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  if (threadIdx.x == 0 && (int)blockIdx.x < n) out[blockIdx.x] = (int32_t)(x & 0xf);
}

}  // namespace

extern "C" int ll_decode_attention_xcc_probe(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                             int64_t head_dim, int64_t max_len_in_batch,
                                             int32_t* out, int64_t out_len, hipStream_t stream) {
  LL_CHECK_ARG(out != nullptr && batch > 0 && kv_heads > 0 && q_heads % kv_heads == 0 &&
                   (head_dim == 64 || head_dim == 128) && max_len_in_batch > 0,
               "ll_decode_attention_xcc_probe: bad arguments");
  const int nsplit = choose_nsplit((int)batch, (int)kv_heads, max_len_in_batch, head_dim);
  const int groups = (int)((batch + 7) / 8);
  const int64_t grid = (int64_t)groups * 8 * kv_heads * nsplit;
  LL_CHECK_ARG(out_len >= grid, "ll_decode_attention_xcc_probe: out holds %lld of %lld entries",
               (long long)out_len, (long long)grid);
  const int64_t tiles = (max_len_in_batch + kTT - 1) / kTT;
  const size_t slots_cap = (size_t)((tiles + nsplit - 1) / nsplit) * kTT;
  const size_t lds =
      (head_dim == 128 ? TileGeom<128>::MAIN_B : TileGeom<64>::MAIN_B) + slots_cap * 4;
  hipLaunchKernelGGL(xcc_probe_kernel, dim3((unsigned)grid), dim3(kWaves * 64), lds, stream, out,
                     (int)grid);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    ll_set_error("HIP launch failed: %s", hipGetErrorString(e));
    return LL_ERR_HIP;
  }
  return (int)grid;
}

extern "C" int ll_decode_attention_set_same_launch_merge(int enable) {
  const int old = g_same_launch_merge.exchange(enable ? 1 : 0);
  return old;
}

extern "C" int ll_decode_attention_split_count(int64_t batch, int64_t kv_heads, int64_t head_dim,
                                               int64_t max_len_in_batch) {
  return choose_nsplit((int)batch, (int)kv_heads, max_len_in_batch, head_dim);
}

extern "C" int64_t ll_decode_attention_workspace_size(int64_t batch, int64_t q_heads,
                                                      int64_t kv_heads, int64_t head_dim,
                                                      int64_t max_len_in_batch) {
  return workspace_bytes_for(batch, q_heads, kv_heads, head_dim, max_len_in_batch);
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
  LL_CHECK_ARG(max_len_in_batch >= 0 && max_len_in_batch <= INT32_MAX,
               "ll_decode_attention: max_len_in_batch %lld out of range",
               (long long)max_len_in_batch);
  if (batch == 0) return LL_OK;
  DecodeArgs a = {};
  a.q = q; a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.k = k_cache; a.k_st = k_stride_tok; a.k_sh = k_stride_head;
  a.v = v_cache; a.v_st = v_stride_tok; a.v_sh = v_stride_head;
  a.r2t = req_to_tokens; a.r2t_s = req_to_tokens_stride;
  a.req_idx = b_req_idx; a.req64 = req_idx_i64;
  a.seq_len = b_seq_len; a.len64 = seq_len_i64;
  a.out = out; a.o_sb = out_stride_b; a.o_sh = out_stride_h;
  a.B = (int)batch; a.H = (int)q_heads; a.KVH = (int)kv_heads; a.G = (int)(q_heads / kv_heads);
  a.units = a.B * a.KVH;
  a.max_len = (int)max_len_in_batch;
  a.slots_cap = 0;
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

  return launch_mfma(a, head_dim, dtype, false, max_len_in_batch, workspace, workspace_bytes,
                     stream);
}

// ---------------------------------------------------------------- no-allocation variant
// ll_decode_attention_noalloc runs ll_decode_attention with a library-owned
// scratch buffer in place of the caller's workspace: a file-scope device array
// that every GPU the library runs on holds until the process ends. In host
// code `scratch` names a host-side stand-in, not the device array, so the
// device address is looked up once per device (hipGetSymbolAddress, with that
// device current) and only that address is ever passed to kernels.
namespace {

constexpr int64_t kNoAllocScratchBytes = 4 << 20;  // split tickets + partials
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's scratch array, looked up on the first
// call on the device (or by ll_decode_attention_noalloc_init). Nothing is
// written to the array here: as a zero-initialised device global it starts
// with every split ticket at zero, and every call leaves them at zero, so the
// lookup queues no work on any stream (it may happen while a caller captures
// a graph).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    ll_set_error("ll_decode_attention_noalloc: no usable current device (%s)",
                 hipGetErrorString(e));
    return LL_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      ll_set_error("ll_decode_attention_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                   hipGetErrorString(e));
      return LL_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return LL_OK;
}

}  // namespace

extern "C" int ll_decode_attention_noalloc_init(void) {
  void* p = nullptr;
  return scratch_for_current_device(&p);
}

extern "C" int64_t ll_decode_attention_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int ll_decode_attention_noalloc(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
    int64_t k_stride_tok, int64_t k_stride_head, const void* v_cache, int64_t v_stride_tok,
    int64_t v_stride_head, const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
    const void* b_req_idx, int req_idx_i64, const void* b_seq_len, int seq_len_i64, void* out,
    int64_t out_stride_b, int64_t out_stride_h, int64_t batch, int64_t q_heads, int64_t kv_heads,
    int64_t head_dim, int64_t max_len_in_batch, float sm_scale, int dtype, hipStream_t stream) {
  LL_CHECK_ARG(batch >= 0 && kv_heads > 0 && q_heads > 0 && head_dim > 0,
               "ll_decode_attention_noalloc: bad shape");
  const int64_t need =
      batch == 0 ? 0 : workspace_bytes_for(batch, q_heads, kv_heads, head_dim, max_len_in_batch);
  LL_CHECK_ARG(need <= kNoAllocScratchBytes,
               "ll_decode_attention_noalloc: this shape needs %lld bytes of split partials, more "
               "than the %lld-byte scratch; use ll_decode_attention with a workspace",
               (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_for_current_device(&ws);
    if (rc != LL_OK) return rc;
  }
  return ll_decode_attention(q, q_stride_b, q_stride_h, k_cache, k_stride_tok, k_stride_head,
                             v_cache, v_stride_tok, v_stride_head, req_to_tokens,
                             req_to_tokens_stride, b_req_idx, req_idx_i64, b_seq_len, seq_len_i64,
                             out, out_stride_b, out_stride_h, batch, q_heads, kv_heads, head_dim,
                             max_len_in_batch, sm_scale, dtype, ws, need > 0 ? kNoAllocScratchBytes : 0,
                             stream);
}

namespace {

int rope_attention_impl(const LLPartials& qkv, const void* qkv_bias, const void* positions,
                        int positions_i64, const void* cos_table, const void* sin_table,
                        int64_t table_row_stride, int cs_dtype, const int32_t* new_slots,
                        void* k_cache, int64_t k_stride_tok, int64_t k_stride_head, void* v_cache,
                        int64_t v_stride_tok, int64_t v_stride_head, const int32_t* req_to_tokens,
                        int64_t req_to_tokens_stride, const void* b_req_idx, int req_idx_i64,
                        const void* b_seq_len, int seq_len_i64, void* out, int64_t out_stride_b,
                        int64_t out_stride_h, int64_t batch, int64_t q_heads, int64_t kv_heads,
                        int64_t head_dim, int64_t max_len_in_batch, float sm_scale, int dtype,
                        void* workspace, int64_t workspace_bytes, const float* q_static,
                        int8_t* q_out, int64_t ldq, float* q_scale, uint32_t* error_word,
                        hipStream_t stream) {
  LL_CHECK_ARG((q_out == nullptr) == (q_scale == nullptr) &&
                   (q_out == nullptr || (out_stride_h == head_dim && ldq >= q_heads * head_dim)),
               "ll_decode_attention_rope_splitk: q_out needs q_scale, contiguous output rows "
               "and ldq >= q_heads * head_dim");
  LL_CHECK_ARG(qkv.p && positions && cos_table && sin_table && new_slots && k_cache && v_cache &&
                   req_to_tokens && b_req_idx && b_seq_len && out,
               "ll_decode_attention_rope_splitk: null pointer");
  LL_CHECK_ARG(qkv.splits >= 1, "ll_decode_attention_rope_splitk: qkv_splits must be >= 1");
  LL_CHECK_ARG(cs_dtype == LL_F32, "ll_decode_attention_rope_splitk: cos/sin tables must be fp32");
  LL_CHECK_ARG(kv_heads > 0 && q_heads % kv_heads == 0 && q_heads / kv_heads <= 16,
               "ll_decode_attention_rope_splitk: needs q_heads = G * kv_heads with G <= 16");
  LL_CHECK_ARG((dtype == LL_BF16 || dtype == LL_F16) && (head_dim == 128 || head_dim == 64),
               "ll_decode_attention_rope_splitk: bf16/fp16 with head_dim 64 or 128 only "
               "(other shapes: ll_rope_kv_scatter_splitk + ll_decode_attention)");
  LL_CHECK_ARG(k_stride_tok % 8 == 0 && k_stride_head % 8 == 0 && v_stride_tok % 8 == 0 &&
                   v_stride_head % 8 == 0 &&
                   (((uintptr_t)qkv.p | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0),
               "ll_decode_attention_rope_splitk: K/V strides must be multiples of 8 elements, "
               "partials and caches 16 B aligned");
  LL_CHECK_ARG(max_len_in_batch >= 0 && max_len_in_batch <= INT32_MAX,
               "ll_decode_attention_rope_splitk: max_len_in_batch %lld out of range",
               (long long)max_len_in_batch);
  if (batch == 0) return LL_OK;
  DecodeArgs a = {};
  a.k = k_cache; a.k_st = k_stride_tok; a.k_sh = k_stride_head;
  a.v = v_cache; a.v_st = v_stride_tok; a.v_sh = v_stride_head;
  a.r2t = req_to_tokens; a.r2t_s = req_to_tokens_stride;
  a.req_idx = b_req_idx; a.req64 = req_idx_i64;
  a.seq_len = b_seq_len; a.len64 = seq_len_i64;
  a.out = out; a.o_sb = out_stride_b; a.o_sh = out_stride_h;
  a.B = (int)batch; a.H = (int)q_heads; a.KVH = (int)kv_heads; a.G = (int)(q_heads / kv_heads);
  a.units = a.B * a.KVH;
  a.max_len = (int)max_len_in_batch;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.qkv = qkv;
  a.qkv.sstride = batch * (q_heads + 2 * kv_heads) * head_dim;
  a.qkv_bias = qkv_bias;
  a.pos = positions; a.pos64 = positions_i64;
  a.cos_tab = (const float*)cos_table; a.sin_tab = (const float*)sin_table;
  a.tab_stride = table_row_stride;
  a.new_slots = new_slots;
  a.qout = q_out; a.ldq = ldq; a.qscale = q_scale; a.qstatic = q_static;
  // the split merge's wait follows the decode step's spin setting and
  // reports a give-up in the step's error word
  const int spin = ll_decode_spin_setting();
  a.unit_spin = spin < 0 ? -spin : spin;
  a.unit_never = spin < 0 ? 1 : 0;
  a.err = error_word;
  return launch_mfma(a, head_dim, dtype, true, max_len_in_batch, workspace, workspace_bytes,
                     stream);
}

}  // namespace

extern "C" int ll_decode_attention_rope_splitk(
    const float* qkv_part, int qkv_splits, const void* qkv_bias, const void* positions,
    int positions_i64, const void* cos_table, const void* sin_table, int64_t table_row_stride,
    int cs_dtype, const int32_t* new_slots, void* k_cache, int64_t k_stride_tok,
    int64_t k_stride_head, void* v_cache, int64_t v_stride_tok, int64_t v_stride_head,
    const int32_t* req_to_tokens, int64_t req_to_tokens_stride, const void* b_req_idx,
    int req_idx_i64, const void* b_seq_len, int seq_len_i64, void* out, int64_t out_stride_b,
    int64_t out_stride_h, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t max_len_in_batch, float sm_scale, int dtype, void* workspace,
    int64_t workspace_bytes, uint32_t* error_word, hipStream_t stream) {
  return rope_attention_impl(ll_partials_f32(qkv_part, qkv_splits, 0), qkv_bias, positions,
                             positions_i64, cos_table, sin_table, table_row_stride, cs_dtype,
                             new_slots, k_cache, k_stride_tok, k_stride_head, v_cache, v_stride_tok,
                             v_stride_head, req_to_tokens, req_to_tokens_stride, b_req_idx,
                             req_idx_i64, b_seq_len, seq_len_i64, out, out_stride_b, out_stride_h,
                             batch, q_heads, kv_heads, head_dim, max_len_in_batch, sm_scale, dtype,
                             workspace, workspace_bytes, nullptr, nullptr, 0, nullptr, error_word,
                             stream);
}

extern "C" int ll_decode_attention_rope_splitk_i32(
    const int32_t* qkv_part, int qkv_splits, const float* s_tok, const void* s_ch, int s_ch_dtype,
    const void* qkv_bias, const void* positions, int positions_i64, const void* cos_table,
    const void* sin_table, int64_t table_row_stride, int cs_dtype, const int32_t* new_slots,
    void* k_cache, int64_t k_stride_tok, int64_t k_stride_head, void* v_cache,
    int64_t v_stride_tok, int64_t v_stride_head, const int32_t* req_to_tokens,
    int64_t req_to_tokens_stride, const void* b_req_idx, int req_idx_i64, const void* b_seq_len,
    int seq_len_i64, void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t batch,
    int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t max_len_in_batch,
    float sm_scale, int dtype, void* workspace, int64_t workspace_bytes, const float* q_static,
    int8_t* q_out, int64_t ldq, float* q_scale, uint32_t* error_word, hipStream_t stream) {
  LL_CHECK_ARG(s_tok && s_ch, "ll_decode_attention_rope_splitk_i32: null scale pointer");
  LL_CHECK_ARG(s_ch_dtype == LL_F32 || s_ch_dtype == LL_F16 || s_ch_dtype == LL_BF16,
               "ll_decode_attention_rope_splitk_i32: bad scale dtype %d", s_ch_dtype);
  LL_CHECK_ARG(((uintptr_t)s_ch) % 4 == 0,
               "ll_decode_attention_rope_splitk_i32: s_ch must be 4 B aligned");
  LLPartials P = {qkv_part, qkv_splits, 0, s_tok, s_ch, s_ch_dtype, 1};
  return rope_attention_impl(P, qkv_bias, positions, positions_i64, cos_table, sin_table,
                             table_row_stride, cs_dtype, new_slots, k_cache, k_stride_tok,
                             k_stride_head, v_cache, v_stride_tok, v_stride_head, req_to_tokens,
                             req_to_tokens_stride, b_req_idx, req_idx_i64, b_seq_len, seq_len_i64,
                             out, out_stride_b, out_stride_h, batch, q_heads, kv_heads, head_dim,
                             max_len_in_batch, sm_scale, dtype, workspace, workspace_bytes,
                             q_static, q_out, ldq, q_scale, error_word, stream);
}
