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
//     with fp32 state (a row's running maximum moves only when a tile's
//     maximum passes it by more than 2^8, so that the output rows are
//     rescaled about once per work item), and O^T += V^T . P^T with P
//     rounded to the KV dtype;
//   * one barrier per tile.
#include <algorithm>
#include <type_traits>

#include "ll_common.h"

namespace {

constexpr int kBK = 64;   // keys per tile
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left free (gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int kVmcntZero = 0x0F70;

constexpr int kStages = 4;  // LDS ring depth (K/V tiles)
// A row's running maximum (exp2 domain) moves only when a tile's maximum
// passes it by more than this: the probabilities then stay at most 2^8
// (exact range in fp32 and in the 16-bit P fed to P.V)
constexpr float kLazyMax = 8.0f;

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

// s_waitcnt vmcnt(0) with the Q fragments as operands: their loads are
// issued before it and their values are defined by it
__device__ __forceinline__ void q_wait_tie(bf16x8 (&q)[8]) {
  asm volatile("s_waitcnt vmcnt(0)"
               : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]),
                 "+v"(q[6]), "+v"(q[7])::"memory");
}
__device__ __forceinline__ void q_wait_tie(bf16x8 (&q)[4]) {
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3])::"memory");
}
__device__ __forceinline__ void q_wait_tie(f16x8 (&q)[8]) {
  asm volatile("s_waitcnt vmcnt(0)"
               : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]),
                 "+v"(q[6]), "+v"(q[7])::"memory");
}
__device__ __forceinline__ void q_wait_tie(f16x8 (&q)[4]) {
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3])::"memory");
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

// Work items: one per (query-row block, request, KV head, head group). Item
// numbers ("virtual blocks") put the head groups of one (row block, request,
// KV head) 8 apart, so that they take workgroups of one XCD (workgroup i runs
// on XCD i mod 8, up to a constant rotation) and read its K/V tiles through
// one L2, and put the longest (last) row blocks first. The grid is
// persistent (P workgroups, P a multiple of 16, at most 64 passes):
// workgroup w takes item jP + w on even passes j and, on odd passes, the
// items of its XCD in reverse slot order, (j + 1)P - 8 (w / 8 + 1) + w mod 8
// (a snake over the slots that keeps item mod 8 = w mod 8, so that the items
// of one (request, KV head) stay on one XCD whenever 8 divides the items per
// row block).
__device__ __forceinline__ int64_t fa_item_of_pass(int j, int P, int w) {
  return (j & 1) ? (int64_t)(j + 1) * P - 8 * ((w >> 3) + 1) + (w & 7) : (int64_t)j * P + w;
}

// The fields of the first loads (lengths, shared prefixes, start offsets,
// request rows and the grid geometry) come as scalar arguments ahead of the
// PrefillArgs block: gfx950 preloads leading scalar kernel arguments into
// SGPRs at dispatch, so those loads do not wait for the argument block's
// load. idx64: bit 0 lengths, 1 shared, 2 starts, 3 request rows are int64.
// nv: virtual blocks (items, valid or not) of the launch.
template <typename T, int D, int WPH>
__global__ __launch_bounds__(512) void prefill_attn_fa_kernel(
    const void* __restrict__ p_len, const void* __restrict__ p_shared,
    const void* __restrict__ p_start, const void* __restrict__ p_rid, int idx64, int nblk, int B,
    int KVH, int G, int nv, PrefillArgs a) {
  typedef typename Vec8<T>::type V8;
  typedef FaGeom<D> FG;
  typedef FaShape<WPH> SH;
  constexpr int QB = 1;  // 32-row query blocks per wave
  constexpr int DS = D / 16;  // k-steps of S^T = K . Q^T
  constexpr int DB = D / 32;  // 32-row d blocks of O^T
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int HP = (G + SH::HPW - 1) / SH::HPW;  // head groups per KV head
  const int P = (int)gridDim.x, w = (int)blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, hf = lane >> 5;

  // The item table, built by every wave alike in one round trip: lane j
  // holds the workgroup's item of pass j (its request's values, its KV head
  // and head group, its first query row, key count and tile count). An item
  // is valid when its row block starts inside its request's query rows.
  int it_L = 0, it_S = 0, it_blk0 = 0, it_kvend = 1, it_nt = 0, it_kvh = 0, it_hp = 0;
  int64_t it_start = 0, it_rid = 0;
  bool it_ok = false;
  {
    const int64_t vb = fa_item_of_pass(lane, P, w);  // vb >= nv for every pass past the last
    const int units = nblk * B * KVH;
    if (vb < nv && ((int)(vb >> 3) / HP) * 8 + (int)(vb & 7) < units) {
      const int unit = ((int)(vb >> 3) / HP) * 8 + (int)(vb & 7);
      const int b = (unit / KVH) % B;
      // every per-request value in one round trip
      const int64_t L = ll_load_idx(p_len, b, idx64 & 1);
      const int64_t S = p_shared ? ll_load_idx(p_shared, b, (idx64 >> 1) & 1) : 0;
      it_start = ll_load_idx(p_start, b, (idx64 >> 2) & 1);
      it_rid = ll_load_idx(p_rid, b, (idx64 >> 3) & 1);
      const int64_t blk0 = (int64_t)(nblk - 1 - unit / (KVH * B)) * SH::BQ;
      if (blk0 < L - S) {
        // token indices within a request fit in 32 bits (lengths below 2^31)
        it_ok = true;
        it_L = (int)L;
        it_S = (int)S;
        it_blk0 = (int)blk0;
        it_kvend = (int)min(L, blk0 + SH::BQ + S);  // keys of the item
        it_nt = (it_kvend + kBK - 1) / kBK;
        it_kvh = unit % KVH;
        it_hp = (int)(vb >> 3) % HP;
      }
    }
  }
  const uint64_t items = __builtin_amdgcn_ballot_w64(it_ok);
  if (items == 0) return;  // uniform over the workgroup
  int ntot = it_ok ? it_nt : 0;  // tiles of the workgroup's stream
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ntot += __shfl_xor(ntot, o, 64);
  ntot = __builtin_amdgcn_readfirstlane(ntot);
  auto next_item = [&](int k) -> int {  // the valid item after pass k (64: none)
    const uint64_t rest = k >= 63 ? 0 : items & (~(uint64_t)0 << (k + 1));
    return rest ? (int)__builtin_ctzll(rest) : 64;
  };
  auto rl = [&](int v, int k) -> int { return __builtin_amdgcn_readlane(v, k); };
  auto rl64 = [&](int64_t v, int k) -> int64_t {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint64_t)v, k);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)((uint64_t)v >> 32), k);
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };

  // This wave's view of an item: its head, its first query row and whether
  // it has rows there, the keys its rows see, the request's query start.
  struct WaveItem {
    int64_t start;
    int h, row0, qlast, S, Lm1, kv_end;
    bool ok;
  };
  auto wave_item = [&](int k) -> WaveItem {
    WaveItem r;
    const int L = rl(it_L, k), S = rl(it_S, k), blk0 = rl(it_blk0, k);
    const int gh = SH::HPW * rl(it_hp, k) + wave / SH::WPH;  // head within the KV head's group
    r.start = rl64(it_start, k);
    r.h = rl(it_kvh, k) * G + (gh < G ? gh : 0);
    r.row0 = blk0 + SH::RW * (wave % SH::WPH);
    r.qlast = L - S - 1;
    r.ok = gh < G && r.row0 <= r.qlast;
    r.S = S;
    r.Lm1 = L - 1;
    r.kv_end = (int)min((int64_t)L, (int64_t)r.row0 + SH::RW + S);
    return r;
  };
  // Q^T fragments (B operand: column = query row row0 + l32, clamped into the
  // request; k-slots = d 16 s + 8 hf .. +7), in registers for the whole item
  V8 qreg[DS];
  auto load_q = [&](const WaveItem& it) {
    const int r = min(it.row0 + l32, it.qlast);
    const T* qp = (const T*)a.q + (it.start + r) * a.q_st + (int64_t)it.h * a.q_sh + 8 * hf;
#pragma unroll
    for (int s = 0; s < DS; ++s) qreg[s] = *(const V8*)(qp + 16 * s);
  };

  // The workgroup's items run as one stream of 64-key tiles. K and V tiles
  // go from the pool straight into an NST-stage LDS ring
  // (global_load_lds_dwordx4, no VGPR staging); the slot ids that address
  // them are DMA'd likewise, by every wave into a ring of its own, NST - 1
  // tiles before the tile's K/V copies. Per stream tile x every wave issues
  // one group: its K/V copies of tile x + NST - 1 and its slot ids of tile
  // x + 2 NST - 2, so that NST - 1 tiles are in flight while tile x is
  // computed, across item boundaries too (the next item's first tiles load
  // under the current item's last ones). Past the stream's end the groups
  // repeat the last item's last key into stages nothing reads, so that
  // every iteration has the same copies in flight.
  constexpr int NST = kStages;
  constexpr int RPI = 64 / FG::CH;                     // rows per DMA instruction
  constexpr int IPW = kBK * FG::ROWB / 1024 / SH::NW;  // K (and V) instructions per wave per tile
  constexpr int KVC = 2 * IPW;                         // K and V
  static_assert(IPW >= 1 && IPW * SH::NW * 1024 == kBK * FG::ROWB, "tile rows over the waves");
  static_assert(NST == 4, "the waits below are written for 4 stages");
  char* wslots = smem + NST * FG::STAGE_B + wave * (NST * kBK * 4);
  const int dr = lane / FG::CH, dp = lane % FG::CH;

  // The copy cursors: the item (pass) and tile of the next group's copies,
  // with that item's addresses (refreshed only when a cursor moves to the
  // next item, so that an iteration's scalar work stays small: the scalar
  // unit serves all eight waves of the CU). Past the stream's end each
  // stays on the last item's last tile.
  struct SlotCursor {
    int k, u, nt, last_key;
    const int32_t* row;
  };
  struct KvCursor {
    int k, left;  // tiles of the item still to copy, the next one included
    const T* kb;
    const T* vb;
  };
  auto slot_at = [&](SlotCursor& c, int k) {
    c.k = k;
    c.u = 0;
    c.nt = rl(it_nt, k);
    c.last_key = rl(it_kvend, k) - 1;
    c.row = a.r2t + rl64(it_rid, k) * a.r2t_s;
  };
  auto kv_at = [&](KvCursor& c, int k) {
    c.k = k;
    c.left = rl(it_nt, k);
    const int kvh = rl(it_kvh, k);
    c.kb = (const T*)a.k + (int64_t)kvh * a.k_sh;
    c.vb = (const T*)a.v + (int64_t)kvh * a.v_sh;
  };
  auto slot_next = [&](SlotCursor& c) {
    if (++c.u == c.nt) {
      const int k2 = next_item(c.k);
      if (k2 < 64) slot_at(c, k2); else c.u = c.nt - 1;
    }
  };
  auto kv_next = [&](KvCursor& c) {
    if (--c.left == 0) {
      const int k2 = next_item(c.k);
      if (k2 < 64) kv_at(c, k2); else c.left = 1;
    }
  };
  const int k_first = (int)__builtin_ctzll(items);
  // slot ids of cursor c's tile (keys 64 u + lane, clamped) -> ring entry x % NST
  auto slot_copy = [&](int x, const SlotCursor& c) {
    dma4(c.row + min(c.u * kBK + lane, c.last_key), wslots + (x % NST) * (kBK * 4));
  };
  // this wave's K and V rows of cursor c's tile (slot ids in ring entry
  // x % NST) -> stage x % NST
  auto kv_copy = [&](int x, const KvCursor& c) {
    char* kl = smem + (x % NST) * FG::STAGE_B;
    char* vl = kl + FG::K_B;
    const int32_t* sl = (const int32_t*)(wslots + (x % NST) * (kBK * 4));
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int ii = wave * IPW + i;
      const int r = ii * RPI + dr;  // the LDS chunk position dp of row r holds chunk swz(dp, r)
      const int64_t slot = sl[r];
      dma16(c.kb + slot * a.k_st + 8 * FG::kswz(dp, r), kl + ii * 1024);
      dma16(c.vb + slot * a.v_st + 8 * FG::vswz(dp, r), vl + ii * 1024);
    }
  };

  f32x16 acc[DB][QB];
  // a row's running maximum (the same in its two lanes) and the sum of its
  // probabilities over the keys of this lane's half-wave
  float m_run[QB], l_run[QB];
  auto reset = [&]() {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) acc[db][qb] = (f32x16){};
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      m_run[qb] = -INFINITY;
      l_run[qb] = 0.f;
    }
  };
  reset();

  WaveItem cur = wave_item(k_first);
  load_q(cur);
  // slot ids of stream tiles 0 .. NST-2, then (every load so far landed, Q
  // fragments included: a real s_waitcnt, which the compiler's own wait
  // insertion accounts for) the groups of iterations -NST+1 .. -1
  SlotCursor cs;
  slot_at(cs, k_first);
  KvCursor ck;
  kv_at(ck, k_first);
#pragma unroll
  for (int x = 0; x < NST - 1; ++x) {
    slot_copy(x, cs);
    slot_next(cs);
  }
  __builtin_amdgcn_s_waitcnt(kVmcntZero);
#pragma unroll
  for (int x = 0; x < NST - 1; ++x) {
    kv_copy(x, ck);
    kv_next(ck);
    slot_copy(x + NST - 1, cs);
    slot_next(cs);
  }

  // S^T[key 32 kb + 8 g + 4 hf + i][query 32 qb + l32] of the current tile in
  // sacc[kb][qb][4 g + i]; the tile's row maxima (exp2 domain) over this
  // half-wave's keys in m_cand
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
    const bool need_mask = t0 + kBK - 1 > min(cur.row0 + cur.S, cur.Lm1);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (need_mask) {
        // last key this row sees, relative to the tile (rows past the
        // request see every key of it)
        const int lim = min(cur.row0 + 32 * qb + l32 + cur.S, cur.Lm1) - t0;
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
      m_cand[qb] = tmax * a.scale_log2;  // this half-wave's keys only
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
      l_run[qb] += psum;  // this half-wave's keys; the halves add up at the store
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
  // acc[db][qb][4 g + i] = O^T[d = 32 db + 8 g + 4 hf + i][query row0 + 32 qb + l32]
  auto store_rows = [&](const WaveItem& it) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int r = it.row0 + 32 * qb + l32;
      if (r > it.qlast) continue;
      const float inv = 1.0f / (l_run[qb] + __shfl_xor(l_run[qb], 32, 64));
      T* op = (T*)a.o + (it.start + r) * a.o_st + (int64_t)it.h * a.o_sh + 4 * hf;
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
  };

  // the next item's Q rows are pulled into L2 ahead of its first tile: one
  // 4-byte DMA per lane into this wave's 256-byte sink (never read), lane i
  // touching 128-byte line i % LPR of row i / LPR of the wave's 32 rows
  char* wsink = smem + NST * FG::STAGE_B + SH::NW * (NST * kBK * 4) + wave * 256;
  auto prefetch_q = [&](const WaveItem& it) {
    constexpr int LPR = FG::ROWB / 128;  // 128-byte lines per Q row
    const int r = min(it.row0 + (lane / LPR) % SH::RW, it.qlast);
    const T* qp = (const T*)a.q + (it.start + r) * a.q_st + (int64_t)it.h * a.q_sh + 64 * (lane % LPR);
    dma4(qp, wsink);
  };

  // iterations whose copies a full wait (at an item's first tile, before
  // that iteration's copies) already covered: after it in iteration y the
  // copies of tiles up to y + NST - 2 and the slot ids they read are in
  int covered = 0;
  int cc_k = k_first, cc_u = 0, cc_nt = rl(it_nt, k_first);  // item (pass) and tile computed
  WaveItem done = cur;  // at an item's first tile: the item whose rows acc holds
  for (int x = 0; x < ntot; ++x) {
    // Otherwise, at the top of iteration x only the groups of iterations
    // x-NST+2 .. x-1 may be in flight (2 slot copies and 2 K/V groups; the
    // groups are issued in every iteration), besides older output stores
    // and newer Q prefetches: vector memory operations complete in issue
    // order, so both only make the wait longer.
    if (covered > 0) --covered; else vm_wait<(NST - 2) + 2 * KVC>();
    // every wave's copies of tile x are in; every wave is done with tile
    // x - 1, whose stage the copies of tile x + NST - 1 refill
    lds_barrier();
    if (cc_u == 0 && x > 0) {
      // An item's first tile (the first item's Q came with the prologue):
      // its Q fragments, from L2, and the wait for them, before this
      // iteration's copies (the wait covers the copies in flight, which
      // were issued a tile or more ago). The loads and the wait stay in one
      // branch and the fragments pass through the wait as operands: the
      // compiler then sees nothing pending across the loop's back edge (it
      // would otherwise wait for every copy in flight before each scores).
      load_q(cur);
      q_wait_tie(qreg);
      covered = NST - 2;
      // the previous item's rows, then a fresh softmax state
      if (done.ok) store_rows(done);
      reset();
    }
    kv_copy(x + NST - 1, ck);
    kv_next(ck);
    slot_copy(x + 2 * NST - 2, cs);
    slot_next(cs);
    const int t0 = cc_u * kBK, buf = x % NST;
    const bool work = cur.ok && t0 < cur.kv_end;
    const bool last = cc_u + 1 == cc_nt;
    if (work) scores(t0, buf);
    if (last) {
      const int k2 = next_item(cc_k);
      if (k2 < 64) prefetch_q(wave_item(k2));
    }
    if (work) {
      // running maxima, moved only when a row of the wave meets a tile
      // maximum more than kLazyMax above its own (the first tile always):
      // until then the probabilities exp2(s - m_run) stay below 2^kLazyMax,
      // and the output rows and sums are rescaled about once per item
      // instead of at nearly every tile
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        if (__builtin_amdgcn_ballot_w64(m_cand[qb] > m_run[qb] + kLazyMax)) {
          // both halves of a row (its two lanes) take the row's maximum
          const float m_new =
              fmaxf(m_run[qb], fmaxf(m_cand[qb], __shfl_xor(m_cand[qb], 32, 64)));
          const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
          m_run[qb] = m_new;
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db) acc[db][qb] *= alpha;
        }
      }
      accumulate(buf);
    }
    if (!last) {
      ++cc_u;
    } else {
      const int k2 = next_item(cc_k);
      if (k2 < 64) {  // (past the last item's last tile the loop ends)
        done = cur;
        cur = wave_item(k2);
        cc_k = k2;
        cc_u = 0;
        cc_nt = rl(it_nt, k2);
      }
    }
  }
  // no copy may still be writing this workgroup's LDS when it ends
  vm_wait<0>();
  if (cur.ok) store_rows(cur);
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
  const int64_t nv = (int64_t)ll_cdiv(units, 8) * 8 * ll_cdiv(a.G, 8 / wph);  // work items
  LL_CHECK_ARG(nv < ((int64_t)1 << 31), "ll_prefill_attention: %lld work items (max 2^31 - 1)",
               (long long)nv);
  // persistent grid: one workgroup per CU (the LDS ring takes the whole CU),
  // a multiple of 16 so that the head groups of a (row block, request, KV
  // head) share an XCD on the reversed passes too; more when the items
  // would need more than 64 passes
  int cus = 0;
  const int rc = ll_device_cus(&cus);
  if (rc != LL_OK) return rc;
  int64_t P = std::max<int64_t>(16, cus / 16 * 16);
  if (ll_cdiv(nv, P) > 64) P = (int64_t)ll_cdiv(ll_cdiv(nv, 64), 16) * 16;
  P = std::min(P, nv);
  const dim3 grid((unsigned)P);
  const dim3 block(512);
  auto launch = [&](auto tag, auto dtag) {
    typedef decltype(tag) T;
    constexpr int D = decltype(dtag)::value;
    constexpr size_t lds = kStages * FaGeom<D>::STAGE_B + 8 * kStages * kBK * 4 + 8 * 256;
    const int idx64 = (a.len64 ? 1 : 0) | (a.shared64 ? 2 : 0) | (a.start64 ? 4 : 0) |
                      (a.req64 ? 8 : 0);
    if (wph == 2)
      hipLaunchKernelGGL((prefill_attn_fa_kernel<T, D, 2>), grid, block, lds, stream, a.seq_len,
                         a.shared, a.start_loc, a.req_idx, idx64, a.nblk, a.B, a.KVH, a.G, (int)nv,
                         a);
    else
      hipLaunchKernelGGL((prefill_attn_fa_kernel<T, D, 4>), grid, block, lds, stream, a.seq_len,
                         a.shared, a.start_loc, a.req_idx, idx64, a.nblk, a.B, a.KVH, a.G, (int)nv,
                         a);
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
