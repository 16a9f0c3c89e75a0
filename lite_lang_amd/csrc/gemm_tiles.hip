// Prefill projections (M > 64 rows): Y[M, N] = X[M, K] . W[N, K]^T on MFMA,
// gfx950. Replaces the torch.addmm / torch.mm products of the reference's
// prefill (litelang/models/qwen2/layer/transformer_layer.py:80,82,95-109,193)
// for bf16/fp16, and is the int8 x int8 -> int32 product of the W8A8 runtime
// (the reference's SmoothQuant module has no forward, quantize/smooth_quant/
// layer.py:19-59).
//
// One workgroup (8 waves, two per SIMD) per CU computes 256 x 256 output
// tiles one after the other (a persistent grid):
//   * stages of 64 bytes of K per row (32 bf16/fp16 or 64 int8) for the
//     tile's 256 weight rows and 256 activation rows (32 KB) are copied
//     global -> LDS with global_load_lds_dwordx4 (no VGPR staging) into a
//     ring of five stage buffers (160 KB), four stages in flight ahead of
//     the one being multiplied; the ring runs on from one tile into the
//     next, so no tile after the first waits for its first stages;
//   * a finished tile's outputs are stored with buffer stores that nothing
//     waits for until the ring's own waits reach them, a few stages into
//     the next tile;
//   * the 16-byte chunks of every LDS row are XOR-swizzled (tile_swz) so
//     the MFMA operand reads (16 rows x 16 B per 16 lanes) hit distinct
//     banks;
//   * each wave multiplies 128 weight rows by 64 activation rows with
//     v_mfma_f32_32x32x16_bf16 (v_mfma_i32_32x32x32_i8 for int8) as
//     C^T = W . X^T: the weight rows are the MFMA's row operand, so every
//     lane ends with runs of 4 consecutive output columns of one token row
//     (8-byte stores) in 8 accumulator blocks of 32 x 32. The second wave
//     on each SIMD issues while the first waits on LDS or the barrier (one
//     wave per SIMD reaches about 150 B/clk of LDS reads per CU, two about
//     240);
//   * the grid is XCD-aware: the workgroups the dispatcher deals to one XCD
//     take a contiguous range of tiles in groups of 1, 2 or 4 row tiles by
//     shape (tile_group_m), round robin, so tiles sharing activation or
//     weight rows run together on one L2.
// Epilogues: the model dtype with an optional bias; SiLU_and_Mul of a
// gate/up weight interleaved in 64-row blocks (ll_gemm_interleave_gate_up),
// with the rounding sequence of ll_silu_and_mul; int8 sums dequantised as
// fp32(acc) * s_tok[m] * fp32(s_ch[n]) (+ bias) as ll_dequant_splitk does;
// raw int32 sums.
#include <algorithm>
#include <atomic>

#include "ll_common.h"

namespace {

constexpr int kT = 256;        // output tile: 256 activation rows x 256 weight rows
constexpr int kRB = 64;        // bytes of K per row per stage
constexpr int kStageB = 2 * kT * kRB;  // 32 KB: weight rows, then activation rows
constexpr int kNst = 5;        // stage buffers (160 KB of LDS)
constexpr int kWaves = 8;      // two per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kPW = 4;         // 32-row weight blocks per wave (128 rows: wave column wn of 2)
constexpr int kQX = 2;         // 32-row activation blocks per wave (64 rows: wave row wm of 4)
constexpr int kNMf = kPW * kQX;  // MFMAs per wave per k-step
constexpr int kDmaW = 2 * kT * kRB / 16 / kThreads;  // 16-byte copies per lane per stage
static_assert(2 * 32 * kPW == kT && 4 * 32 * kQX == kT && kWaves == 8, "wave grid 2 x 4");
static_assert(kDmaW == 4, "copy geometry: 4 instructions of 16 rows per wave per stage");

enum { EPI_STORE = 0, EPI_SILU = 1, EPI_DEQ = 2, EPI_DEQ_SILU = 3, EPI_I32 = 4 };

typedef float f32x16v __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
template <typename T> struct TileOp;
template <> struct TileOp<__bf16> { typedef bf16x8 V; typedef f32x16v Acc; };
template <> struct TileOp<_Float16> { typedef f16x8 V; typedef f32x16v Acc; };
template <> struct TileOp<int8_t> { typedef i32x4 V; typedef i32x16 Acc; };

// 32 x 32 output block, 16 bf16/fp16 (32 int8) of K per instruction: lane l
// supplies row (or column) l % 32 and the 16-byte K chunk l / 32
__device__ __forceinline__ f32x16v tile_mma(bf16x8 a, bf16x8 b, f32x16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16v tile_mma(f16x8 a, f16x8 b, f32x16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ i32x16 tile_mma(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// 16 B global -> LDS copy of one lane (lane i lands at lds + 16 i); kept out of
// the templates (a dependent call of this builtin drops the host launch stub).
__device__ __forceinline__ void tile_dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

template <int N_> __device__ __forceinline__ void tile_vm_wait() {
  static_assert(N_ >= 0 && N_ < 64, "vmcnt is a 6-bit counter");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

// Barrier that waits for this wave's LDS reads only (its own copies were
// waited for with tile_vm_wait; __syncthreads would also drain the copies of
// the stages in flight).
__device__ __forceinline__ void tile_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

struct TileArgs {
  const char* X; int64_t ldx_b;   // activation rows (K contiguous), row stride in bytes
  const char* W; int64_t ldw_b;   // weight rows [N][K] (EPI_SILU*: interleaved gate/up)
  int M, N, K_b;                  // K in bytes
  int tiles_m, tiles_n;
  int group_m;                    // row tiles per group of the tile order (tile_group_m)
  void* Y; int64_t ldy;           // output, row stride in elements of the output type
  int y_bytes;                    // bytes from Y to the end of its last row (< 2^31)
  const void* bias;               // [N] in the model dtype, or null
  const float* s_tok;             // int8: activation scale per row [M]
  const void* s_ch; int s_ch_dtype;  // int8: weight scale per channel [N]
};

// Swizzle of the 16-byte chunks of 64-byte LDS row r (an involution on
// 0..3): chunk c of row r sits at chunk c ^ ((r / 4) % 4). Measured with
// ds_read_b128 over the fragment pattern (32 rows x one chunk per 32
// lanes): about 205 B/clk per CU, as for contiguous reads, against 116 B/clk
// for a swizzle on (r / 2) ^ (r / 8) and 63 B/clk unswizzled.
__device__ __forceinline__ int tile_swz(int r) { return (r >> 2) & 3; }
// LDS byte offset of chunk c (16 B) of tile row r within a stage half
__device__ __forceinline__ int tile_lds_off(int r, int c) { return r * kRB + ((c ^ tile_swz(r)) << 4); }

// Output tile (m0, n0) of tile t of the grouped order: groups of group_m row
// tiles, each group's column tiles in order with its row tiles innermost.
__device__ __forceinline__ void tile_coords(const TileArgs& a, int t, int& m0, int& n0) {
  const int gsz = a.group_m * a.tiles_n;
  const int grp = t / gsz, rin = t - grp * gsz;
  const int gm = min(a.group_m, a.tiles_m - grp * a.group_m);
  m0 = (grp * a.group_m + rin % gm) * kT;
  n0 = (rin / gm) * kT;
}

// Row tiles per group of the tile order, by shape class, as measured on the
// 3B prefill projections at M = 24,000 (group sizes 1, 2, 4 and 8, libraries
// interleaved, best of 4 rounds): wide outputs (gate/up, 86 column tiles)
// 4 (1788 us against 1813 with 2 and 1886-1898 with 1 or 8); long K
// (down_proj, 172 stages) 1 (916 against 953 with 2); the narrow short-K
// shapes (qkv, o_proj) level at every size (2).
int tile_group_m(int64_t tiles_n, int64_t nk) {
  if (tiles_n >= 32) return 4;
  if (nk >= 128) return 1;
  return 2;
}

// Buffer store of 4 consecutive outputs. A lane whose offset is kTileNoStore
// (beyond the buffer's size) stores nothing, so every wave issues the same
// number of store instructions for every tile, edges included: the copy
// ring's vmcnt waits count them. The empty asm keeps the compiler from
// merging stores, which would change that count.
constexpr uint32_t kTileNoStore = 0x80000000u;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <typename TO>
__device__ __forceinline__ void tile_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, const TO (&o)[4]) {
  typedef TO V4 __attribute__((ext_vector_type(4)));
  const V4 v = {o[0], o[1], o[2], o[3]};
  if constexpr (sizeof(TO) == 2) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
  }
  asm volatile("" ::: "memory");
}

// Raw bits of the scales of `n` consecutive channels from i (fp32 bits, or a
// zero-extended fp16 / bf16 code; ll_scale_bits_to_f32 converts them). The
// dtype branch is taken once for all the loads, so none waits for another.
template <int n>
__device__ __forceinline__ void tile_scale_bits(const void* s, int dtype, const int (&i)[n],
                                                uint32_t (&b)[n][4]) {
  if (dtype == LL_F32) {
#pragma unroll
    for (int j = 0; j < n; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) b[j][k] = ((const uint32_t*)s)[i[j] + k];
  } else {
#pragma unroll
    for (int j = 0; j < n; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) b[j][k] = ((const uint16_t*)s)[i[j] + k];
  }
}

template <typename T, typename TO, int EPI>
__global__ __launch_bounds__(kThreads, 1) void gemm_tile_kernel(TileArgs a) {
  typedef typename TileOp<T>::V V;
  typedef typename TileOp<T>::Acc Acc;
  constexpr bool kSilu = EPI == EPI_SILU || EPI == EPI_DEQ_SILU;
  constexpr int kStores = kSilu ? 16 : 32;  // store instructions per wave per tile
  extern __shared__ __attribute__((aligned(16))) char smem[];

  // ---- tiles of this workgroup. XCD x (= blockIdx % 8, up to a launch-wide
  // rotation) owns tiles x * per .. x * per + per - 1 of the grouped order;
  // its gridDim / 8 workgroups (one per CU) take them round robin, so the
  // tiles in flight on one XCD at any time are consecutive in that order.
  const int tiles = a.tiles_m * a.tiles_n;
  const int per = (tiles + 7) / 8;
  const int g8 = (int)(gridDim.x >> 3);
  const int t_first = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  const int t_end = min((int)(blockIdx.x & 7) * per + per, tiles);
  if (t_first >= t_end) return;
  const int ntl = (t_end - t_first + g8 - 1) / g8;  // tiles of this workgroup
  const int nk = a.K_b / kRB;                        // stages per tile
  const int total = ntl * nk;                        // stages this workgroup multiplies

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wn = wave & 1, wm = wave >> 1;

  // ---- copy stream: the stages of all of this workgroup's tiles in order,
  // so a tile's first stages are copied while the previous tile is still
  // being multiplied. Instruction u of this wave is copy j = u * 8 + wave of
  // the stage's 32; copy j covers LDS rows 16 * (j % 16) .. + 15 of the
  // weight half (j < 16) or the activation half; lane -> row + l/4, LDS
  // chunk l % 4.
  const int crow = lane >> 2;
  uint32_t soff[kDmaW];  // byte offsets of this lane's copy sources (rows clamped into range)
  auto set_sources = [&](int t) {
    int m0, n0;
    tile_coords(a, t, m0, n0);
#pragma unroll
    for (int u = 0; u < kDmaW; ++u) {
      const int j = u * kWaves + wave;
      const int r = 16 * (j & 15) + crow;
      const int gch = (lane & 3) ^ tile_swz(r);
      if (j < 16) soff[u] = (uint32_t)((int64_t)min(n0 + r, a.N - 1) * a.ldw_b + gch * 16);
      else soff[u] = (uint32_t)((int64_t)min(m0 + r, a.M - 1) * a.ldx_b + gch * 16);
    }
  };
  set_sources(t_first);
  int iss_j = 0, iss_ks = 0, iss_buf = 0;  // tile (local index), stage and ring buffer of the next copies
  // Copies past the last tile repeat its last stage (in bounds, never read),
  // so every wave's vmcnt arithmetic is the same in every iteration.
  auto issue = [&]() {
    const int ks = iss_j < ntl ? iss_ks : nk - 1;
#pragma unroll
    for (int u = 0; u < kDmaW; ++u) {
      const int j = u * kWaves + wave;
      char* dst = smem + iss_buf * kStageB + (j >> 4) * (kT * kRB) + (j & 15) * 1024;
      tile_dma16((j < 16 ? a.W : a.X) + (int64_t)ks * kRB + soff[u], dst);
    }
    iss_buf = iss_buf == kNst - 1 ? 0 : iss_buf + 1;
    if (iss_j < ntl && ++iss_ks == nk) {
      iss_ks = 0;
      if (++iss_j < ntl) set_sources(t_first + iss_j * g8);
    }
  };

  Acc acc[kPW][kQX];
  auto zero_acc = [&]() {
#pragma unroll
    for (int p = 0; p < kPW; ++p)
#pragma unroll
      for (int q = 0; q < kQX; ++q)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[p][q][e] = 0;
  };
  zero_acc();

  const int lr = lane & 31, lc = lane >> 5;
  const int wrow = wn * 128 + lr, xrow = wm * 64 + lr;
  const int c0 = lc, c1 = 2 + lc;  // LDS chunks of k-step 0 and 1 for this lane
  V fw[2][kPW], fx[2][kQX];
  auto frag_w = [&](int buf, int c, int p) {
    return *(const V*)(smem + buf * kStageB + tile_lds_off(wrow + 32 * p, c));
  };
  auto frag_x = [&](int buf, int c, int q) {
    return *(const V*)(smem + buf * kStageB + kT * kRB + tile_lds_off(xrow + 32 * q, c));
  };
  auto read_stage = [&](int g) {
    const int buf = g % kNst;
#pragma unroll
    for (int p = 0; p < kPW; ++p) fw[0][p] = frag_w(buf, c0, p);
#pragma unroll
    for (int q = 0; q < kQX; ++q) fx[0][q] = frag_x(buf, c0, q);
#pragma unroll
    for (int p = 0; p < kPW; ++p) fw[1][p] = frag_w(buf, c1, p);
#pragma unroll
    for (int q = 0; q < kQX; ++q) fx[1][q] = frag_x(buf, c1, q);
  };
  auto compute = [&]() {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < kNMf; ++i)
        acc[i / kQX][i % kQX] = tile_mma(fw[kk][i / kQX], fx[kk][i % kQX], acc[i / kQX][i % kQX]);
  };

  // ---- epilogue of tile ep_j: acc[p][q][4g + i] = C[m][n] with
  //   m = m0 + wm*64 + 32q + l % 32,  n = n0 + wn*128 + 32p + 8g + 4(l / 32) + i
  const __amdgpu_buffer_rsrc_t yres =
      __builtin_amdgcn_make_buffer_rsrc(a.Y, (short)0, a.y_bytes, 0x00020000);
  int ep_j = 0;
  auto epilogue = [&]() {
    int m0, n0;
    tile_coords(a, t_first + ep_j * g8, m0, n0);
    ++ep_j;
    const int mrow = m0 + wm * 64 + lr;
    // The per-row and per-column factors are all loaded before the first
    // store, so the wave waits for them (and for the copies in flight ahead
    // of them) once, not once per store.
    float st[kQX];
#pragma unroll
    for (int q = 0; q < kQX; ++q) {
      st[q] = 1.f;
      if constexpr (EPI == EPI_DEQ || EPI == EPI_DEQ_SILU) st[q] = a.s_tok[min(mrow + 32 * q, a.M - 1)];
    }
    if constexpr (!kSilu) {
      typedef TO V4 __attribute__((ext_vector_type(4)));
      const bool has_bias = EPI != EPI_I32 && a.bias != nullptr;
      const int ncol = n0 + wn * 128 + 4 * lc;
      // weight blocks p per pass: the dequantising epilogue's scales take 4
      // registers per column group, so it makes two passes
      constexpr int kPass = EPI == EPI_DEQ ? 2 : kPW;
#pragma unroll
      for (int p0 = 0; p0 < kPW; p0 += kPass) {
        int nl[kPass * 4];  // in-range column groups for the loads
#pragma unroll
        for (int j = 0; j < kPass * 4; ++j) {
          const int n = ncol + 32 * (p0 + j / 4) + 8 * (j % 4);
          nl[j] = n < a.N ? n : 0;
        }
        uint32_t sb[kPass * 4][4];
        if constexpr (EPI == EPI_DEQ) tile_scale_bits<kPass * 4>(a.s_ch, a.s_ch_dtype, nl, sb);
        V4 bv[kPass][4];
        if (has_bias) {
#pragma unroll
          for (int j = 0; j < kPass * 4; ++j) bv[j / 4][j % 4] = *(const V4*)((const TO*)a.bias + nl[j]);
        }
#pragma unroll
        for (int pp = 0; pp < kPass; ++pp)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int p = p0 + pp;
            const int n = ncol + 32 * p + 8 * g;
            const bool n_ok = n < a.N;
#pragma unroll
            for (int q = 0; q < kQX; ++q) {
              const int m = mrow + 32 * q;
              TO o[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                if constexpr (EPI == EPI_I32) {
                  o[i] = (TO)acc[p][q][4 * g + i];
                } else if constexpr (EPI == EPI_DEQ) {
                  // the product is rounded before the bias is added (no fused
                  // multiply-add), as in ll_dequant_splitk followed by the add
                  const float sc = ll_scale_bits_to_f32(sb[4 * pp + g][i], a.s_ch_dtype);
                  float v = (float)acc[p][q][4 * g + i] * st[q] * sc;
                  asm volatile("" : "+v"(v));
                  if (has_bias) v += ll_to_f32(bv[pp][g][i]);
                  o[i] = ll_from_f32<TO>(v);
                } else {
                  o[i] = ll_from_f32<TO>(acc[p][q][4 * g + i] +
                                         (has_bias ? ll_to_f32(bv[pp][g][i]) : 0.f));
                }
              }
              const uint32_t off = (n_ok && m < a.M)
                                       ? (uint32_t)(((int64_t)m * a.ldy + n) * (int64_t)sizeof(TO))
                                       : kTileNoStore;
              tile_store4<TO>(yres, off, o);
            }
          }
      }
    } else {
      // gate/up interleaved in 64-row blocks: this wave's rows 0..63 (p < 2)
      // are gate channels c, rows 64..127 (p >= 2) the up channels c, with
      // c = n0 / 2 + wn * 64 + 32 (p % 2) + 8g + 4(l / 32) + i; N = 2 I
      const int I = a.N / 2;
      const int cbase = n0 / 2 + wn * 64 + 4 * lc;
      // scales of the gate channels (groups 0..7) and the up channels (8..15)
      uint32_t sb[16][4];
      if constexpr (EPI == EPI_DEQ_SILU) {
        int cl[16];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int c = cbase + 32 * (j / 4) + 8 * (j % 4);
          cl[j] = c < I ? c : 0;
          cl[8 + j] = I + cl[j];
        }
        tile_scale_bits<16>(a.s_ch, a.s_ch_dtype, cl, sb);
      }
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c = cbase + 32 * p + 8 * g;
          const bool c_ok = c < I;
#pragma unroll
          for (int q = 0; q < kQX; ++q) {
            const int m = mrow + 32 * q;
            TO o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float gs, us;
              if constexpr (EPI == EPI_DEQ_SILU) {
                gs = (float)acc[p][q][4 * g + i] * st[q] *
                     ll_scale_bits_to_f32(sb[4 * p + g][i], a.s_ch_dtype);
                us = (float)acc[p + 2][q][4 * g + i] * st[q] *
                     ll_scale_bits_to_f32(sb[8 + 4 * p + g][i], a.s_ch_dtype);
              } else {
                gs = acc[p][q][4 * g + i];
                us = acc[p + 2][q][4 * g + i];
              }
              const float gv = ll_to_f32(ll_from_f32<TO>(gs));
              const float u = ll_to_f32(ll_from_f32<TO>(us));
              const TO sv = ll_from_f32<TO>(ll_silu_f32(gv));
              o[i] = ll_from_f32<TO>(u * ll_to_f32(sv));
            }
            const uint32_t off = (c_ok && m < a.M)
                                     ? (uint32_t)(((int64_t)m * a.ldy + c) * (int64_t)sizeof(TO))
                                     : kTileNoStore;
            tile_store4<TO>(yres, off, o);
          }
        }
    }
  };

  // Ping-pong schedule. Waves 0-3 (group A) and 4-7 (group B) hold one
  // wave of each SIMD (the dispatcher places wave w on SIMD w % 4). Time is
  // cut into phases separated by workgroup barriers; in phase 2g group A
  // multiplies stage g (of this workgroup's stage sequence) from its
  // registers while group B reads its fragments of stage g from LDS and
  // issues its half of the copies of stage g + 4, and in phase 2g + 1 the
  // roles swap (B multiplies stage g, A reads stage g + 1 and issues its
  // half of stage g + 4). Each SIMD's MFMA pipe so always has one wave with
  // a run of 16 independent MFMAs while the other wave's LDS reads and
  // copies proceed. Ring invariants (five buffers, stage t in buffer t % 5):
  //   * stage t lands before the barrier that ends phase 2t - 2 (A waits
  //     vmcnt(8) at the end of its compute phase, B vmcnt(12) after
  //     issuing), so A's reads in phase 2t - 1 and B's in phase 2t see it;
  //   * the copies of stage t + 5 go to stage t's buffer in phases 2t + 2
  //     and 2t + 3, after the barrier that ends B's last read of stage t
  //     (phase 2t, closed by lgkmcnt(0)).
  // A wave writes a finished tile's outputs in its first memory phase after
  // the tile's last stage (A: phase 2g + 1, B: phase 2g + 2), before that
  // phase's copies, and does not wait for the stores: the vmcnt waits of
  // the next phases allow kStores more operations when stores were issued
  // after the copies they wait for (a count at or below the exact one is
  // always safe; vmcnt retires in issue order).
  static_assert(kNst == 5 && kDmaW == 4, "the ping-pong wait counts assume 5 buffers, 4 copies");
  static_assert(12 + kStores < 64, "vmcnt is a 6-bit counter");
  const bool group_a = wave < 4;
  // prologue: B issues its halves of stages 0..3, A of stages 0..2; stage 0
  // lands; A reads stage 0 and issues its half of stage 3 (phase -1)
  issue();
  issue();
  issue();
  if (group_a) {
    tile_vm_wait<8>();
  } else {
    issue();
    tile_vm_wait<12>();
  }
  tile_barrier();
  if (group_a) {
    read_stage(0);
    issue();
  }
  tile_barrier();
  // sched_barrier keeps every instruction inside its phase (MFMAs touch no
  // memory, so nothing else stops the scheduler moving them across barriers)
  int cks = 0;        // stage within its tile of the stage being multiplied
  int last_ep = -8;   // iteration of this wave's last epilogue
  if (group_a) {
    for (int g = 0; g < total; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      compute();                 // phase 2g: stage g
      __builtin_amdgcn_sched_barrier(0);
      // own copies of stage g + 1 landed; they were issued in iteration
      // g - 3, before the stores of an epilogue in iteration g - 2 or g - 1
      if (g - last_ep <= 2) tile_vm_wait<8 + kStores>();
      else tile_vm_wait<8>();
      tile_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (cks == nk - 1) {       // phase 2g + 1
        epilogue();
        zero_acc();
        last_ep = g;
      }
      read_stage(g + 1);
      issue();                   // stage g + 4
      __builtin_amdgcn_sched_barrier(0);
      tile_barrier();
      cks = cks == nk - 1 ? 0 : cks + 1;
    }
  } else {
    for (int g = 0; g < total; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      if (g > 0 && cks == 0) {   // phase 2g: the previous tile's outputs
        epilogue();
        zero_acc();
        last_ep = g;
      }
      read_stage(g);
      issue();                   // stage g + 4
      __builtin_amdgcn_sched_barrier(0);
      // own copies of stage g + 1 landed; they were issued in iteration
      // g - 3, before the stores of an epilogue in iteration g - 2 .. g
      if (g - last_ep <= 2) tile_vm_wait<12 + kStores>();
      else tile_vm_wait<12>();
      tile_barrier();
      __builtin_amdgcn_sched_barrier(0);
      compute();                 // phase 2g + 1: stage g
      __builtin_amdgcn_sched_barrier(0);
      tile_barrier();
      cks = cks == nk - 1 ? 0 : cks + 1;
    }
    epilogue();
  }
  __builtin_amdgcn_sched_barrier(0);
  tile_vm_wait<0>();
}

// Interleave a [gate; up] weight ([2I, K], I % 128 == 0) into 64-row blocks:
// out row R of tile R / 256: block (R % 256) / 64 alternates gate and up rows
// of channels (R / 256) * 128 + ((R % 256) / 128) * 64 + R % 64.
__global__ void interleave_gate_up_kernel(const u32x4* __restrict__ W, int64_t ldw16,
                                          u32x4* __restrict__ out, int64_t row16, int I,
                                          int64_t total) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= total) return;
  const int64_t R = u / row16, c = u - R * row16;
  const int64_t t = R / 256, r = R % 256;
  const int64_t blk = r / 64, ch = t * 128 + (blk / 2) * 64 + (r % 64);
  const int64_t src = (blk % 2 == 0) ? ch : I + ch;
  out[u] = W[src * ldw16 + c];
}

// The kernel addresses its copy sources with 32-bit row offsets and its
// stores with 31-bit buffer offsets: the weight must span less than 4 GiB
// (checked by the entry points), and the activation and output rows are
// launched in chunks whose spans fit (and whose stage count per workgroup
// fits an int).
template <typename T, typename TO, int EPI>
int launch_tiles(const TileArgs& a0, hipStream_t stream) {
  int cus = 0;
  const int rc = ll_device_cus(&cus);
  if (rc != LL_OK) return rc;
  const int64_t yrow_b = a0.ldy * (int64_t)sizeof(TO);
  const int64_t tiles_n = ll_cdiv(a0.N, kT), nk = a0.K_b / kRB;
  const int64_t rows_x = (((int64_t)1 << 32) - 2 * kRB) / a0.ldx_b;
  const int64_t rows_y = (((int64_t)1 << 31) - 1) / yrow_b;
  const int64_t rows_s = ((int64_t)INT32_MAX / nk) * 8 / tiles_n * kT;
  const int64_t max_rows = std::min(rows_x, std::min(rows_y, rows_s));
  LL_CHECK_ARG(max_rows >= 1, "gemm tiles: output rows or K too large for one launch");
  const int64_t chunk =
      max_rows >= a0.M ? a0.M : (max_rows >= kT ? (max_rows / kT) * kT : max_rows);
  for (int64_t mo = 0; mo < a0.M; mo += chunk) {
    TileArgs a = a0;
    a.X += mo * a0.ldx_b;
    a.Y = (char*)a0.Y + mo * yrow_b;
    if (a0.s_tok != nullptr) a.s_tok = a0.s_tok + mo;
    a.M = (int)(a0.M - mo < chunk ? a0.M - mo : chunk);
    a.y_bytes = (int)((a.M - 1) * yrow_b + a.N * (int64_t)sizeof(TO));
    a.tiles_m = ll_cdiv(a.M, kT);
    a.tiles_n = (int)tiles_n;
    a.group_m = tile_group_m(tiles_n, nk);
    const int64_t per = ((int64_t)a.tiles_m * a.tiles_n + 7) / 8;
    const int64_t grid = 8 * std::min<int64_t>(per, std::max(1, cus / 8));
    hipLaunchKernelGGL((gemm_tile_kernel<T, TO, EPI>), dim3((unsigned)grid), dim3(kThreads),
                       (size_t)kNst * kStageB, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      ll_set_error("HIP launch failed: %s", hipGetErrorString(e));
      return LL_ERR_HIP;
    }
  }
  return LL_OK;
}

// ldx, ldw in elements of es bytes; ldy in elements of Y, whose rows hold
// ny outputs (N, or N / 2 for the gate/up epilogues).
int check_tile_args(const char* name, const void* X, int64_t ldx, const void* W, int64_t ldw,
                    const void* Y, int64_t ldy, int64_t ny, int64_t M, int64_t N, int64_t K_b,
                    int64_t es) {
  LL_CHECK_ARG(X && W && Y, "%s: null pointer", name);
  LL_CHECK_ARG(M > 0 && N > 0 && N % 4 == 0 && K_b > 0 && K_b % kRB == 0,
               "%s: needs M > 0, N %% 4 == 0 and K a multiple of %lld (M=%lld N=%lld K=%lld)", name,
               (long long)(kRB / es), (long long)M, (long long)N, (long long)(K_b / es));
  LL_CHECK_ARG(ldx * es >= K_b && ldw * es >= K_b && ldy >= ny,
               "%s: row strides shorter than the rows (ldx=%lld ldw=%lld K=%lld, ldy=%lld for "
               "%lld outputs per row)",
               name, (long long)ldx, (long long)ldw, (long long)(K_b / es), (long long)ldy,
               (long long)ny);
  LL_CHECK_ARG((ldx * es) % 16 == 0 && (ldw * es) % 16 == 0 &&
                   (((uintptr_t)X | (uintptr_t)W) % 16) == 0,
               "%s: X and W rows must be 16 B aligned", name);
  LL_CHECK_ARG(M <= INT32_MAX && N <= INT32_MAX && K_b <= INT32_MAX, "%s: shape too large", name);
  LL_CHECK_ARG((N - 1) * ldw * es + K_b < ((int64_t)1 << 32) && ldx * es < ((int64_t)1 << 31),
               "%s: the weight must span less than 4 GiB", name);
  return LL_OK;
}

TileArgs make_args(const void* X, int64_t ldx_b, const void* W, int64_t ldw_b, int64_t M,
                   int64_t N, int64_t K_b, void* Y, int64_t ldy) {
  TileArgs a = {};
  a.X = (const char*)X; a.ldx_b = ldx_b;
  a.W = (const char*)W; a.ldw_b = ldw_b;
  a.M = (int)M; a.N = (int)N; a.K_b = (int)K_b;
  a.Y = Y; a.ldy = ldy;
  return a;
}

}  // namespace

int ll_device_cus(int* cus_out) {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    ll_set_error("hipGetDevice failed");
    return LL_ERR_HIP;
  }
  int n = dev >= 0 && dev < 64 ? cache[dev].load(std::memory_order_relaxed) : 0;
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      ll_set_error("hipDeviceGetAttribute(MultiprocessorCount) failed");
      return LL_ERR_HIP;
    }
    if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  }
  *cus_out = n;
  return LL_OK;
}

extern "C" int ll_gemm_tiled_supported(int64_t M, int64_t N, int64_t K, int dtype) {
  if (dtype != LL_BF16 && dtype != LL_F16) return 0;
  return M > 0 && N > 0 && N % 4 == 0 && K > 0 && (K * 2) % kRB == 0;
}

extern "C" int ll_gemm_tiled(const void* X, int64_t ldx, const void* W, int64_t ldw,
                             const void* bias, void* Y, int64_t ldy, int64_t M, int64_t N,
                             int64_t K, int dtype, hipStream_t stream) {
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "ll_gemm_tiled: bf16 or fp16 only");
  const int rc = check_tile_args("ll_gemm_tiled", X, ldx, W, ldw, Y, ldy, N, M, N, K * 2, 2);
  if (rc != LL_OK) return rc;
  LL_CHECK_ARG(ldy % 4 == 0 && ((uintptr_t)Y) % 8 == 0, "ll_gemm_tiled: Y rows must be 8 B aligned");
  LL_CHECK_ARG(((uintptr_t)bias) % 8 == 0, "ll_gemm_tiled: bias must be 8 B aligned");
  TileArgs a = make_args(X, ldx * 2, W, ldw * 2, M, N, K * 2, Y, ldy);
  a.bias = bias;
  if (dtype == LL_BF16) return launch_tiles<__bf16, __bf16, EPI_STORE>(a, stream);
  return launch_tiles<_Float16, _Float16, EPI_STORE>(a, stream);
}

extern "C" int ll_gemm_interleave_gate_up(const void* W, int64_t ldw, int64_t I, int64_t K,
                                          int64_t elem_bytes, void* out, hipStream_t stream) {
  LL_CHECK_ARG(W && out, "ll_gemm_interleave_gate_up: null pointer");
  LL_CHECK_ARG(I > 0 && I % 128 == 0 && K > 0 && (K * elem_bytes) % 16 == 0 &&
                   (ldw * elem_bytes) % 16 == 0 && (elem_bytes == 1 || elem_bytes == 2),
               "ll_gemm_interleave_gate_up: needs I %% 128 == 0 and 16 B rows");
  const int64_t row16 = K * elem_bytes / 16, total = 2 * I * row16;
  hipLaunchKernelGGL(interleave_gate_up_kernel, dim3((unsigned)ll_cdiv(total, 256)), dim3(256), 0,
                     stream, (const u32x4*)W, ldw * elem_bytes / 16, (u32x4*)out, row16, (int)I,
                     total);
  LL_RETURN_LAUNCH();
}

extern "C" int ll_gemm_gate_up_silu_tiled(const void* X, int64_t ldx, const void* W_il,
                                          int64_t M, int64_t I, int64_t K, int dtype, void* Y,
                                          int64_t ldy, hipStream_t stream) {
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "ll_gemm_gate_up_silu_tiled: bf16 or fp16 only");
  LL_CHECK_ARG(I % 128 == 0, "ll_gemm_gate_up_silu_tiled: I must be a multiple of 128");
  const int rc = check_tile_args("ll_gemm_gate_up_silu_tiled", X, ldx, W_il, K, Y, ldy, I, M,
                                 2 * I, K * 2, 2);
  if (rc != LL_OK) return rc;
  LL_CHECK_ARG(ldy % 4 == 0 && ((uintptr_t)Y) % 8 == 0,
               "ll_gemm_gate_up_silu_tiled: Y rows must be 8 B aligned");
  TileArgs a = make_args(X, ldx * 2, W_il, K * 2, M, 2 * I, K * 2, Y, ldy);
  if (dtype == LL_BF16) return launch_tiles<__bf16, __bf16, EPI_SILU>(a, stream);
  return launch_tiles<_Float16, _Float16, EPI_SILU>(a, stream);
}

extern "C" int ll_gemm_i8_tiled(const int8_t* Xq, int64_t ldx, const float* s_tok,
                                const int8_t* Wq, int64_t ldw, const void* s_ch, int s_ch_dtype,
                                const void* bias, void* Y, int64_t ldy, int64_t M, int64_t N,
                                int64_t K, int out_dtype, hipStream_t stream) {
  const int rc = check_tile_args("ll_gemm_i8_tiled", Xq, ldx, Wq, ldw, Y, ldy, N, M, N, K, 1);
  if (rc != LL_OK) return rc;
  LL_CHECK_ARG(out_dtype == LL_BF16 || out_dtype == LL_F16 || out_dtype == LL_F32,
               "ll_gemm_i8_tiled: bad output dtype %d", out_dtype);
  LL_CHECK_ARG(s_tok && s_ch && (s_ch_dtype == LL_F32 || s_ch_dtype == LL_F16 ||
                                 s_ch_dtype == LL_BF16),
               "ll_gemm_i8_tiled: needs s_tok and s_ch (fp32/fp16/bf16)");
  LL_CHECK_ARG(bias == nullptr || out_dtype != LL_F32,
               "ll_gemm_i8_tiled: a bias needs a 16-bit output dtype");
  LL_CHECK_ARG(ldy % 4 == 0 && ((uintptr_t)Y) % 16 == 0, "ll_gemm_i8_tiled: Y rows must be 16 B aligned");
  LL_CHECK_ARG(((uintptr_t)bias) % 8 == 0, "ll_gemm_i8_tiled: bias must be 8 B aligned");
  TileArgs a = make_args(Xq, ldx, Wq, ldw, M, N, K, Y, ldy);
  a.bias = bias; a.s_tok = s_tok; a.s_ch = s_ch; a.s_ch_dtype = s_ch_dtype;
  if (out_dtype == LL_BF16) return launch_tiles<int8_t, __bf16, EPI_DEQ>(a, stream);
  if (out_dtype == LL_F16) return launch_tiles<int8_t, _Float16, EPI_DEQ>(a, stream);
  return launch_tiles<int8_t, float, EPI_DEQ>(a, stream);
}

extern "C" int ll_gemm_i8_i32_tiled(const int8_t* Xq, int64_t ldx, const int8_t* Wq, int64_t ldw,
                                    int32_t* Y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                                    hipStream_t stream) {
  const int rc = check_tile_args("ll_gemm_i8_i32_tiled", Xq, ldx, Wq, ldw, Y, ldy, N, M, N, K, 1);
  if (rc != LL_OK) return rc;
  LL_CHECK_ARG(ldy % 4 == 0 && ((uintptr_t)Y) % 16 == 0,
               "ll_gemm_i8_i32_tiled: Y rows must be 16 B aligned");
  TileArgs a = make_args(Xq, ldx, Wq, ldw, M, N, K, Y, ldy);
  return launch_tiles<int8_t, int32_t, EPI_I32>(a, stream);
}

// Shapes outside the tile kernel's layout (K not a multiple of 64, unaligned
// rows; small test models): one thread per output, the int8 dot product over
// K in 4-byte steps where the rows allow (v_dot4_i32_i8), exact int32 sums.
__global__ __launch_bounds__(256) void gemm_i8_plain_kernel(const int8_t* __restrict__ X,
                                                            int64_t ldx,
                                                            const int8_t* __restrict__ W,
                                                            int64_t ldw, int32_t* __restrict__ Y,
                                                            int64_t ldy, int M, int N, int K,
                                                            int vec4) {
  const int n = blockIdx.x * 64 + (threadIdx.x & 63);
  const int m = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (m >= M || n >= N) return;
  const int8_t* xr = X + (int64_t)m * ldx;
  const int8_t* wr = W + (int64_t)n * ldw;
  int32_t acc = 0;
  int k = 0;
  if (vec4) {
    for (; k + 4 <= K; k += 4)
      acc = __builtin_amdgcn_sdot4(*(const int32_t*)(xr + k), *(const int32_t*)(wr + k), acc, false);
  }
  for (; k < K; ++k) acc += (int32_t)xr[k] * (int32_t)wr[k];
  Y[(int64_t)m * ldy + n] = acc;
}

extern "C" int ll_gemm_i8_gate_up_silu_tiled(const int8_t* Xq, int64_t ldx, const float* s_tok,
                                             const int8_t* Wq_il, const void* s_ch,
                                             int s_ch_dtype, int64_t M, int64_t I, int64_t K,
                                             int out_dtype, void* Y, int64_t ldy,
                                             hipStream_t stream) {
  LL_CHECK_ARG(I % 128 == 0, "ll_gemm_i8_gate_up_silu_tiled: I must be a multiple of 128");
  const int rc = check_tile_args("ll_gemm_i8_gate_up_silu_tiled", Xq, ldx, Wq_il, K, Y, ldy, I, M,
                                 2 * I, K, 1);
  if (rc != LL_OK) return rc;
  LL_CHECK_ARG(out_dtype == LL_BF16 || out_dtype == LL_F16,
               "ll_gemm_i8_gate_up_silu_tiled: bf16 or fp16 output");
  LL_CHECK_ARG(s_tok && s_ch && (s_ch_dtype == LL_F32 || s_ch_dtype == LL_F16 ||
                                 s_ch_dtype == LL_BF16),
               "ll_gemm_i8_gate_up_silu_tiled: needs s_tok and s_ch (fp32/fp16/bf16)");
  LL_CHECK_ARG(ldy % 4 == 0 && ((uintptr_t)Y) % 8 == 0,
               "ll_gemm_i8_gate_up_silu_tiled: Y rows must be 8 B aligned");
  TileArgs a = make_args(Xq, ldx, Wq_il, K, M, 2 * I, K, Y, ldy);
  a.s_tok = s_tok; a.s_ch = s_ch; a.s_ch_dtype = s_ch_dtype;
  if (out_dtype == LL_BF16) return launch_tiles<int8_t, __bf16, EPI_DEQ_SILU>(a, stream);
  return launch_tiles<int8_t, _Float16, EPI_DEQ_SILU>(a, stream);
}

extern "C" int ll_gemm_i8_i32(const int8_t* Xq, int64_t ldx, const int8_t* Wq, int64_t ldw,
                              int32_t* Y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                              hipStream_t stream) {
  LL_CHECK_ARG(Xq && Wq && Y, "ll_gemm_i8_i32: null pointer");
  LL_CHECK_ARG(M >= 0 && N > 0 && K > 0 && ldx >= K && ldw >= K && ldy >= N,
               "ll_gemm_i8_i32: bad shape (M=%lld N=%lld K=%lld)", (long long)M, (long long)N,
               (long long)K);
  LL_CHECK_ARG(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, "ll_gemm_i8_i32: shape too large");
  if (M == 0) return LL_OK;
  const bool tile = N % 4 == 0 && K % kRB == 0 && ldx % 16 == 0 && ldw % 16 == 0 &&
                    (((uintptr_t)Xq | (uintptr_t)Wq) % 16) == 0 && ldy % 4 == 0 &&
                    ((uintptr_t)Y) % 16 == 0;
  if (tile) return ll_gemm_i8_i32_tiled(Xq, ldx, Wq, ldw, Y, ldy, M, N, K, stream);
  const int vec4 = ldx % 4 == 0 && ldw % 4 == 0 && (((uintptr_t)Xq | (uintptr_t)Wq) % 4) == 0;
  // rows in launches of at most 65535 blocks of 4 (the grid's y limit)
  constexpr int64_t kRowsPerLaunch = 65535 * 4;
  for (int64_t m0 = 0; m0 < M; m0 += kRowsPerLaunch) {
    const int64_t mr = M - m0 < kRowsPerLaunch ? M - m0 : kRowsPerLaunch;
    hipLaunchKernelGGL(gemm_i8_plain_kernel, dim3((unsigned)ll_cdiv(N, 64), (unsigned)ll_cdiv(mr, 4)),
                       dim3(256), 0, stream, Xq + m0 * ldx, ldx, Wq, ldw, Y + m0 * ldy, ldy, (int)mr,
                       (int)N, (int)K, vec4);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      ll_set_error("HIP launch failed: %s", hipGetErrorString(e));
      return LL_ERR_HIP;
    }
  }
  return LL_OK;
}
