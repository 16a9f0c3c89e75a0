// Producer/consumer fusion of the decode step's add + RMSNorm with the QKV
// projection of the next layer, M <= 64 tokens, bf16/fp16, gfx950.
//
// ll_add_rmsnorm_qkv_splitk replaces the pair
//   ll_add_rmsnorm_splitk  (h += sum of the down_proj partials; x = rmsnorm(h))
//   ll_gemm_splitk_packed  (split-K partials of x . Wqkv^T)
// (litelang/models/qwen2/layer/transformer_layer.py:77 and the next layer's
// _InputLayernorm :61 with its q/k/v addmm :95-109) with one launch:
// workgroups 0 .. M-1 each normalise one token row and raise that row's flag;
// every other workgroup owns one (64-row tile, k split) item of the QKV
// product. A wave of an item only ever multiplies its own 16 weight rows, so
// the item's whole weight slice (at most kMaxPer 256-byte chunks per row) is
// loaded straight into registers while the norm runs; after the M row flags
// only the activation chunks (staged in LDS, shared by the four waves) and
// the MFMAs remain. Two launches pay, between the norm and the GEMM, a kernel boundary
// and the GEMM's whole weight round trip.
//
// The k split is this kernel's own (ll_add_rmsnorm_qkv_splits): the fewest
// splits (at most kMaxPer chunks each) whose items, with the norm rows, stay
// within one workgroup per CU (every workgroup resident at once; the dynamic
// LDS request keeps a second one off each CU, so no item shares a CU with a
// norm row). Fewest, because the attention that follows reads every split:
// on the Qwen2.5-3B decode step 4 splits of 4 chunks beat 8 of 2 (128-row
// items), though the shorter items finish this launch sooner. The QKV
// partials therefore sum in a different order
// than ll_gemm_splitk_packed's; the norm outputs are bit-identical to
// ll_add_rmsnorm_splitk's.
//
// No workgroup waits for a workgroup with a higher index, and the dispatcher
// starts workgroups in index order, so the producers are always running or
// done when a consumer waits: the launch cannot deadlock whatever the grid
// size. Each row's data is written with agent-scope (sc1) stores, which reach
// memory before they are acknowledged; the row's flag is stored after that
// acknowledgement; consumers poll the flags with agent-scope loads and read the
// rows with plain loads (nothing of them is cached in their L1/L2 earlier in
// the launch, and kernel boundaries leave the caches coherent). A flag holds
// the call's value *epoch * 256 + tag + 1: the caller makes it differ from
// every earlier call's on the same sync words (a new epoch per decode step,
// the layer index as tag), so flags are never reset and no consumer touches a
// shared counter. Each flag sits in its own 64-byte line. Every poll is
// bounded: a consumer that gives up sets the error word and stores nothing
// (its QKV partials are then missing, so the step's outputs are invalid). The
// decision is each launch's own: an error word left set by an earlier launch
// does not shorten later waits. The word stays set until the host resets it
// (ll_decode_sync_status with reset); ll_argmax_status turns a set word into
// token ids of -1, which is how the runner sees it.
//
// The QKV partials may overwrite the down_proj partials (qkv_part == part):
// every norm workgroup has read its rows of them before it raises its flag,
// and no item stores before it has seen every flag (an item that gave up
// stores nothing at all).
#include "ll_common.h"

#include <atomic>

namespace {

constexpr int kThreads = 512;          // 8 waves (items: 4 working, 4 at the barriers)
constexpr int kRowB = 256;             // bytes of one row chunk (one stage)
constexpr int kKC = 128;               // 16-bit elements per row chunk
constexpr int kSpinMax = 1 << 18;      // polls before a flag wait gives up (default)
constexpr int kMaxLds = 160 * 1024;

template <typename T> struct V8Of;
template <> struct V8Of<__bf16> { typedef bf16x8 type; };
template <> struct V8Of<_Float16> { typedef f16x8 type; };

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------ memory helpers
// Workgroup barrier that waits for LDS operations only (outstanding global
// loads and LDS DMA stay in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}


// Agent-scope stores (sc1: written through to memory before the store is
// acknowledged), for data another workgroup reads later in the same launch.
__device__ __forceinline__ void st_agent_b64(void* p, uint64_t v) {
  asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_agent_b32(void* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_agent_b16(void* p, uint32_t v) {
  asm volatile("global_store_short %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}

template <typename T> __device__ __forceinline__ uint32_t bits16(T v) {
  return (uint32_t)__builtin_bit_cast(unsigned short, v);
}
// four consecutive 16-bit values at p (8-byte aligned when vec)
template <typename T>
__device__ __forceinline__ void st_agent_4(T* p, const T (&y)[4], bool vec, int n_ok) {
  if (vec && n_ok >= 4) {
    const uint64_t v = (uint64_t)bits16(y[0]) | ((uint64_t)bits16(y[1]) << 16) |
                       ((uint64_t)bits16(y[2]) << 32) | ((uint64_t)bits16(y[3]) << 48);
    st_agent_b64(p, v);
  } else {
    for (int e = 0; e < 4 && e < n_ok; ++e) st_agent_b16(p + e, bits16(y[e]));
  }
}

// add + RMSNorm of one row from the split partials with the 512 threads of
// the workgroup, in add_rmsnorm_splitk_kernel's layout and reduction tree
// (thread i takes 4 columns at (512 ps + i) * 4; wave sums, then the 8 wave
// totals in order), so the row is bit-identical to that kernel's. h and out
// are written with agent-scope stores.
template <typename T, int MAXP>
__device__ void norm_row(int row, const float* __restrict__ part, int splits, int M, T* h,
                         int64_t ld_h, const T* __restrict__ gamma, float eps, T* out,
                         int64_t ld_o, int N, float* red) {
  constexpr int PER = 4, OB = 512;
  const int tid = threadIdx.x;
  T* hr = h + (int64_t)row * ld_h;
  T hraw[MAXP][PER], graw[MAXP][PER];
#pragma unroll
  for (int ps = 0; ps < MAXP; ++ps) {
    const int c = min((ps * OB + tid) * PER, N - PER);
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      hraw[ps][e] = hr[c + e];
      graw[ps][e] = gamma[c + e];
    }
  }
  float hv[MAXP][PER];
  float ss = 0.f;
  const bool vec = ((ld_h | ld_o) & 3) == 0;
#pragma unroll
  for (int ps = 0; ps < MAXP; ++ps) {
    const int c = (ps * OB + tid) * PER;
    if (c < N) {
      const f32x4 o = ll_sum_splits4(part, splits, (int64_t)M * N, (int64_t)row * N + c);
      T nh[PER];
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        nh[e] = ll_from_f32<T>(ll_to_f32(hraw[ps][e]) + ll_to_f32(ll_from_f32<T>(o[e])));
        hv[ps][e] = ll_to_f32(nh[e]);
        ss += hv[ps][e] * hv[ps][e];
      }
      st_agent_4(hr + c, nh, vec, N - c);
    }
  }
  const int wave = tid >> 6;
  const float sw = ll_wave_sum(ss);
  if ((tid & 63) == 0) red[wave] = sw;
  lds_barrier();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < 8; ++w) tot += red[w];
  const float denom = sqrtf(tot / (float)N + eps);
  T* orow = out + (int64_t)row * ld_o;
#pragma unroll
  for (int ps = 0; ps < MAXP; ++ps) {
    const int c = (ps * OB + tid) * PER;
    if (c < N) {
      T y[PER];
#pragma unroll
      for (int e = 0; e < PER; ++e)
        y[e] = ll_from_f32<T>(hv[ps][e] / denom * ll_to_f32(graw[ps][e]));
      st_agent_4(orow + c, y, vec, N - c);
    }
  }
  lds_barrier();  // red is reused by the next row
}

// ------------------------------------------------------------ row flags
// sync words: flag i at word kFlagStride * i (i < 64), error word after them.
constexpr int kFlagStride = 16, kMaxFlags = 64, kSyncErr = kFlagStride * kMaxFlags;
constexpr int64_t kSyncBytes = (kSyncErr + 64) * 4;

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Producer epilogue: this workgroup's stores are acknowledged, then its flag.
__device__ __forceinline__ void raise_flag(uint32_t* sync, int idx, uint32_t value) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  if (threadIdx.x == 0)
    __hip_atomic_store(sync + kFlagStride * idx, value, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Consumer: wave 0 polls the n (<= 64) flags, one per lane, until all hold
// `value`, at most spin_max times. Returns, in every thread of the
// workgroup, whether they did; on failure the error word is set.
__device__ __forceinline__ bool wait_flags(uint32_t* sync, int n, uint32_t value, int spin_max,
                                           int* s_ok) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const uint32_t* f = sync + kFlagStride * (lane < n ? lane : 0);
    bool ok = false;
    for (int spins = 0;; ++spins) {
      const uint32_t v = ld_agent(f);
      if (__builtin_amdgcn_ballot_w64(v != value) == 0ull) {
        ok = true;
        break;
      }
      if (spins + 1 >= spin_max) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      *s_ok = ok ? 1 : 0;
      if (!ok)
        __hip_atomic_store(sync + kSyncErr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  lds_barrier();
  return *s_ok != 0;
}

struct NormQkvArgs {
  void* h;
  int64_t ld_h;
  const float* part;       // down_proj partials [splits][M][hidden]
  int splits;
  const void* gamma;
  float eps;
  void* x;                 // [M, hidden], row stride hidden
  const void* wqkv;        // packed QKV weight (ll_gemm_pack, 64-row tiles)
  int tiles, qsplits, per, chunks;
  float* qpart;            // [qsplits][M][nqkv]
  int M, hidden, nqkv;
  uint32_t* sync;
  const uint32_t* epoch;
  uint32_t tag;
  int spin_max;            // polls before a flag wait gives up
  uint32_t skew;           // 0; nonzero only in the test mode (waits that never succeed)
};

constexpr int kMaxPer = 4;        // k chunks per item (16 weight VGPRs each)
constexpr int kMaxItemWgs = 256;  // norm rows + items: one workgroup per CU
constexpr int kMaxSplits = 8;
constexpr int kOneWgLds = 84 * 1024;  // > half the CU's LDS: one workgroup per CU

// The norm rows' first loads (epoch, partials, residual, gamma) take their
// fields from the leading scalar arguments, which gfx950 preloads into SGPRs
// at dispatch, so they do not wait for the load of the argument block.
template <typename T, int MB, int MAXP>
__global__ __launch_bounds__(kThreads) void norm_qkv_kernel(
    const float* __restrict__ part, void* __restrict__ h, int64_t ld_h,
    const void* __restrict__ gamma, const uint32_t* __restrict__ epoch, int M, int splits,
    int hidden, uint32_t tag, NormQkvArgs a) {
  typedef typename V8Of<T>::type V8;
  constexpr int XR = 16 * MB;           // activation rows per chunk (clamped to M - 1)
  constexpr int XB = XR * kRowB;        // LDS bytes per chunk
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __shared__ float red[8];
  __shared__ int s_ok;
  const int w = (int)blockIdx.x;
  const uint32_t value = *epoch * 256u + tag + 1u;
  if (w < M) {
    norm_row<T, MAXP>(w, part, splits, M, (T*)h, ld_h, (const T*)gamma, a.eps, (T*)a.x,
                      (int64_t)hidden, hidden, red);
    raise_flag(a.sync, w, value);
    return;
  }
  const int item = w - a.M;
  const int split = item % a.qsplits, t = item / a.qsplits;
  const int kc0 = split * a.per;
  const int nst = min(a.per, a.chunks - kc0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, j = lane >> 4;
  // waves 0-3 own the tile's 4 x 16 weight rows; waves 4-7 (there for the
  // norm rows' 512 threads) only take part in the workgroup barriers
  const bool work = wave < 4;
  // this wave's weight fragments of every chunk: packed block (kc, t) is the
  // 64 x 256-byte LDS image of the split-K GEMM (row r's 16-byte piece c at
  // r * 256 + (c ^ (r & 15)) * 16); the MFMA A operand of lane (n, j) at
  // k-step s is row 16 wave + n, piece 4 s + j
  const int lr = wave * 16 + n;
  V8 wf[kMaxPer][4];
#pragma unroll
  for (int st = 0; st < kMaxPer; ++st)
    if (st < nst && work) {
      const char* blk = (const char*)a.wqkv + ((int64_t)(kc0 + st) * a.tiles + t) * (64 * kRowB) +
                        lr * kRowB;
#pragma unroll
      for (int s = 0; s < 4; ++s) wf[st][s] = *(const V8*)(blk + (((4 * s + j) ^ (lr & 15)) * 16));
    }
  // an item whose wait gave up stores nothing (the whole workgroup leaves)
  if (!wait_flags(a.sync, a.M, value + a.skew, a.spin_max, &s_ok)) return;
  // activation chunks, all loaded at once (the rows are final: every flag is
  // up) through registers, whose per-CU ingest is faster than LDS DMA's: wave
  // `wave` takes rows 4 MB wave .. +4 MB of each chunk, 16 lanes a row, and
  // stores row r's piece p at LDS r * 256 + (p ^ (r & 15)) * 16 of the chunk's
  // buffer. Rows past M (their MFMA columns are not stored) and chunks past
  // the item's are loaded clamped and not stored: every wave issues the same
  // loads on every path, so the compiler waits for each chunk's loads alone.
  const int xrow0 = 4 * MB * wave + (lane >> 4), p = lane & 15;
  V8 xv_in[kMaxPer][MB];
  if (work) {
#pragma unroll
    for (int st = 0; st < kMaxPer; ++st) {
      const T* g = (const T*)a.x + (int64_t)(kc0 + min(st, nst - 1)) * kKC + p * 8;
#pragma unroll
      for (int e = 0; e < MB; ++e)
        xv_in[st][e] = *(const V8*)(g + (int64_t)min(xrow0 + 4 * e, a.M - 1) * a.hidden);
      __builtin_amdgcn_sched_barrier(0);  // chunk order kept: chunk 0's loads land first
    }
  }
  f32x4 acc[MB];
#pragma unroll
  for (int q = 0; q < MB; ++q) acc[q] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < kMaxPer; ++st)
    if (st < nst) {
      char* xb = smem + st * XB;
      if (work) {
#pragma unroll
        for (int e = 0; e < MB; ++e) {
          const int r = xrow0 + 4 * e;
          if (r < a.M) *(V8*)(xb + r * kRowB + ((p ^ (r & 15)) * 16)) = xv_in[st][e];
        }
      }
      lds_barrier();  // every working wave's rows of chunk st are in
      if (work) {
#pragma unroll
        for (int s = 0; s < kKC / 32; ++s)
#pragma unroll
          for (int q = 0; q < MB; ++q) {
            const int xr = 16 * q + n;
            const V8 xv = *(const V8*)(xb + xr * kRowB + (((4 * s + j) ^ (xr & 15)) * 16));
            acc[q] = mfma16(wf[st][s], xv, acc[q]);
          }
      }
    }
  // acc[q][i] = Y[token 16 q + n][channel 64 t + 16 wave + 4 j + i]; fp32
  // partials qpart[split][m][n], read by the next kernel (plain stores)
  if (!work) return;
  const int ch = t * 64 + wave * 16 + 4 * j;
#pragma unroll
  for (int q = 0; q < MB; ++q) {
    const int tok = 16 * q + n;
    if (tok >= a.M || ch >= a.nqkv) continue;
    *(f32x4*)(a.qpart + ((int64_t)split * a.M + tok) * a.nqkv + ch) = acc[q];
  }
}

template <typename T, int MB>
int launch_norm_qkv(const NormQkvArgs& a, hipStream_t stream) {
  const size_t lds = (size_t)max(kMaxPer * 16 * MB * kRowB, kOneWgLds);
  const dim3 grid((unsigned)(a.M + a.tiles * a.qsplits));
  if (a.hidden <= 2048)
    hipLaunchKernelGGL((norm_qkv_kernel<T, MB, 1>), grid, dim3(kThreads), lds, stream, a.part, a.h,
                       a.ld_h, a.gamma, a.epoch, a.M, a.splits, a.hidden, a.tag, a);
  else
    hipLaunchKernelGGL((norm_qkv_kernel<T, MB, 2>), grid, dim3(kThreads), lds, stream, a.part, a.h,
                       a.ld_h, a.gamma, a.epoch, a.M, a.splits, a.hidden, a.tag, a);
  LL_RETURN_LAUNCH();
}

template <typename T>
int launch_norm_qkv_mb(const NormQkvArgs& a, hipStream_t stream) {
  switch ((a.M + 15) / 16) {
    case 1: return launch_norm_qkv<T, 1>(a, stream);
    case 2: return launch_norm_qkv<T, 2>(a, stream);
    case 3: return launch_norm_qkv<T, 3>(a, stream);
    default: return launch_norm_qkv<T, 4>(a, stream);
  }
}

// The item split: the fewest k splits (at most kMaxSplits) whose items of
// at most kMaxPer chunks, with the M norm rows, stay within one workgroup per
// CU; splits == 0 when none does (the shape is not covered).
struct SplitPlan {
  int tiles, splits, per, chunks;
};
SplitPlan split_plan(int64_t M, int64_t N, int64_t K) {
  SplitPlan p{};
  p.chunks = (int)(K / kKC);
  p.tiles = (int)((N + 63) / 64);
  p.per = kMaxPer < p.chunks ? kMaxPer : p.chunks;
  p.splits = (p.chunks + p.per - 1) / p.per;
  if (p.splits > kMaxSplits || M + (int64_t)p.tiles * p.splits > kMaxItemWgs) p.splits = 0;
  return p;
}

// Polls before a flag wait of the fused decode launches gives up: the
// default, or a bound set by the host. A negative setting -n is a test mode:
// the consumers wait for a flag value no producer writes and give up after n
// polls, so a test sees every wait give up while every kernel still exits
// normally. 0 restores the default.
std::atomic<int> g_spin_max{kSpinMax};
std::atomic<int> g_spin_user{0};  // the setting as given (0: defaults)

}  // namespace

int ll_decode_spin_setting() { return g_spin_user.load(); }

extern "C" int64_t ll_decode_sync_bytes(void) { return kSyncBytes; }

extern "C" int64_t ll_decode_sync_error_offset(void) { return (int64_t)kSyncErr * 4; }

extern "C" int ll_decode_sync_set_spin_limit(int polls) {
  LL_CHECK_ARG(polls > -(1 << 20), "ll_decode_sync_set_spin_limit: bound out of range");
  g_spin_max.store(polls == 0 ? kSpinMax : polls);
  g_spin_user.store(polls);
  return LL_OK;
}

extern "C" int ll_decode_sync_status(void* sync, int reset, hipStream_t stream) {
  LL_CHECK_ARG(sync != nullptr, "ll_decode_sync_status: null sync words");
  uint32_t err = 0;
  if (hipMemcpyAsync(&err, (const char*)sync + kSyncErr * 4, 4, hipMemcpyDeviceToHost, stream) !=
          hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess) {
    ll_set_error("ll_decode_sync_status: copy failed");
    return LL_ERR_HIP;
  }
  if (err != 0u && reset) {
    if (hipMemsetAsync(sync, 0, kSyncBytes, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess) {
      ll_set_error("ll_decode_sync_status: reset failed");
      return LL_ERR_HIP;
    }
  }
  return err != 0u ? 1 : 0;
}

extern "C" int ll_add_rmsnorm_qkv_splits(int64_t M, int64_t hidden, int64_t nqkv) {
  if (M < 1 || M > kMaxFlags || hidden <= 0 || hidden % kKC != 0 || hidden > 4096 || nqkv <= 0 ||
      nqkv % 4 != 0 ||
      ll_gemm_packed_tile_rows(nqkv, hidden) != 64)
    return 0;
  return split_plan(M, nqkv, hidden).splits;
}

extern "C" int ll_add_rmsnorm_qkv_splitk(void* h, int64_t ld_h, const float* part, int splits,
                                         const void* gamma, float eps, void* x,
                                         const void* wqkv_packed, float* qkv_part,
                                         int64_t qkv_part_bytes, int64_t M, int64_t hidden,
                                         int64_t nqkv, int dtype, void* sync,
                                         const uint32_t* epoch, uint32_t tag,
                                         hipStream_t stream) {
  LL_CHECK_ARG(h && part && gamma && x && wqkv_packed && qkv_part && sync && epoch,
               "ll_add_rmsnorm_qkv_splitk: null pointer");
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "ll_add_rmsnorm_qkv_splitk: bf16/fp16 only");
  LL_CHECK_ARG(tag < 256u, "ll_add_rmsnorm_qkv_splitk: tag must be below 256");
  LL_CHECK_ARG(splits >= 1 && ll_add_rmsnorm_qkv_splits(M, hidden, nqkv) > 0,
               "ll_add_rmsnorm_qkv_splitk: shape not covered (M=%lld hidden=%lld nqkv=%lld; "
               "ll_add_rmsnorm_qkv_splits returns 0 for it)",
               (long long)M, (long long)hidden, (long long)nqkv);
  LL_CHECK_ARG(ld_h >= hidden, "ll_add_rmsnorm_qkv_splitk: bad row stride");
  LL_CHECK_ARG((((uintptr_t)part | (uintptr_t)x | (uintptr_t)wqkv_packed | (uintptr_t)qkv_part |
                 (uintptr_t)sync) & 15) == 0,
               "ll_add_rmsnorm_qkv_splitk: misaligned operand");
  const SplitPlan p = split_plan(M, nqkv, hidden);
  LL_CHECK_ARG(qkv_part_bytes >= (int64_t)p.splits * M * nqkv * 4,
               "ll_add_rmsnorm_qkv_splitk: partial buffer too small (need %lld bytes)",
               (long long)((int64_t)p.splits * M * nqkv * 4));
  NormQkvArgs a;
  a.h = h;
  a.ld_h = ld_h;
  a.part = part;
  a.splits = splits;
  a.gamma = gamma;
  a.eps = eps;
  a.x = x;
  a.wqkv = wqkv_packed;
  a.tiles = p.tiles;
  a.qsplits = p.splits;
  a.per = p.per;
  a.chunks = p.chunks;
  a.qpart = qkv_part;
  a.M = (int)M;
  a.hidden = (int)hidden;
  a.nqkv = (int)nqkv;
  a.sync = (uint32_t*)sync;
  a.epoch = epoch;
  a.tag = tag;
  const int spin = g_spin_max.load();
  a.spin_max = spin < 0 ? -spin : spin;
  a.skew = spin < 0 ? 0x80000000u : 0u;
  return dtype == LL_BF16 ? launch_norm_qkv_mb<__bf16>(a, stream)
                          : launch_norm_qkv_mb<_Float16>(a, stream);
}
