// Measurement probes for the paged decode attention's memory floor (no
// counterpart in the reference; bench.py --attention-floor times them).
//
// ll_probe_stream_read: a plain streaming read of `bytes` contiguous bytes,
// 16-byte loads, every workgroup striding over the buffer -- what one launch
// of that size can pull from HBM at all.
//
// ll_probe_kv_gather: the attention's own memory traffic without its
// arithmetic: for every (sequence, KV head, split) of ll_decode_attention's
// grid (same split count, same XCD-aware workgroup order, 8 waves), the
// sequence length and request row, then the split's slot ids, then every K
// and V row of those slots (D * 2 bytes each) -- the same three dependent
// round trips. mode 0 loads the rows into registers, mode 1 copies them into
// LDS (global_load_lds_dwordx4, as the attention does). The rows are folded
// into one word that is stored only if it equals a value no input produces,
// so no load can be dropped.
//
// ll_probe_launch: what a launch costs by itself inside a HIP graph: a grid
// of 512-thread workgroups that does nothing, or writes `write_bytes` with
// 16-byte stores spread over the workgroups (the dirty bytes the launch
// leaves in the L2 for the boundary to write back).
#include "ll_common.h"

namespace {

constexpr int kProbeWaves = 8;

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // four loads in flight per thread per step
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= src[i];
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[0] = x;
}

__global__ __launch_bounds__(512) void launch_probe_kernel(u32x4* __restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * 512;
  for (int64_t i = (int64_t)blockIdx.x * 512 + threadIdx.x; i < n16; i += stride)
    dst[i] = (u32x4){(uint32_t)i, 1u, 2u, 3u};
}

__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

struct GatherArgs {
  const char* k; int64_t k_st, k_sh;  // bytes
  const char* v; int64_t v_st, v_sh;
  const int32_t* r2t; int64_t r2t_s;
  const void* req_idx; int req64;
  const void* seq_len; int len64;
  int B, KVH, nsplit, max_len, row_b;  // row_b = head_dim * element bytes
  uint32_t* sink;
};

// workgroup -> (sequence, KV head, split) exactly as the attention's split
// stage maps them (every workgroup of a sequence on one XCD)
__device__ __forceinline__ void probe_map(int bid, int KVH, int nsplit, int& b, int& kvh, int& split) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per_seq = KVH * nsplit;
  const int k = slot / per_seq, r = slot - k * per_seq;
  b = k * 8 + xcd;
  kvh = r / nsplit;
  split = r - kvh * nsplit;
}

template <int MODE>
__global__ __launch_bounds__(kProbeWaves * 64) void kv_gather_kernel(GatherArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int b, kvh, split;
  probe_map(blockIdx.x, a.KVH, a.nsplit, b, kvh, split);
  if (b >= a.B) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int64_t len = ll_load_idx(a.seq_len, b, a.len64);
  if (len > a.max_len) len = a.max_len;
  const int64_t rid = ll_load_idx(a.req_idx, b, a.req64);
  const int32_t* row = a.r2t + rid * a.r2t_s;
  // the attention's split of the sequence: tile-aligned chunks of 16 tokens
  const int ntiles = (int)((len + 15) / 16);
  const int per = (ntiles + a.nsplit - 1) / a.nsplit;
  const int64_t t0 = (int64_t)min(ntiles, split * per) * 16;
  const int64_t t1 = min(len, (int64_t)min(ntiles, split * per + per) * 16);
  const int cpr = a.row_b / 16;        // 16-byte chunks per row
  const int rpi = 64 / cpr;            // rows per wave instruction
  const int rr = lane / cpr, cc = lane % cpr;
  const char* kb = a.k + (int64_t)kvh * a.k_sh;
  const char* vb = a.v + (int64_t)kvh * a.v_sh;
  u32x4 acc = {0u, 0u, 0u, 0u};
  char* ring = smem + wave * 16 * 1024;
  // every wave takes rpi rows per step, 8 steps (K and V) in flight
  for (int64_t base = t0 + (int64_t)wave * rpi * 4; base < t1; base += (int64_t)kProbeWaves * rpi * 4) {
    int32_t sl[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) sl[u] = row[min(base + u * rpi + rr, t1 - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const char* kp = kb + (int64_t)sl[u] * a.k_st + cc * 16;
      const char* vp = vb + (int64_t)sl[u] * a.v_st + cc * 16;
      if constexpr (MODE == 0) {
        acc ^= *(const u32x4*)kp ^ *(const u32x4*)vp;
      } else {
        dma16(kp, ring + u * 2048);
        dma16(vp, ring + u * 2048 + 1024);
      }
    }
    if constexpr (MODE == 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if constexpr (MODE == 1) acc[0] = *(const uint32_t*)(ring + lane * 16);
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u && split == 12345) a.sink[0] = x;
}

}  // namespace

extern "C" int ll_probe_stream_read(const void* src, int64_t bytes, int64_t workgroups,
                                    uint32_t* sink, hipStream_t stream) {
  LL_CHECK_ARG(src && sink && bytes > 0 && bytes % 16 == 0 && ((uintptr_t)src % 16) == 0,
               "ll_probe_stream_read: needs a 16-byte aligned buffer of 16-byte units");
  LL_CHECK_ARG(workgroups > 0 && workgroups <= (1 << 20), "ll_probe_stream_read: bad grid");
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream,
                     (const u32x4*)src, bytes / 16, sink);
  LL_RETURN_LAUNCH();
}

extern "C" int ll_probe_kv_gather(const void* k_cache, int64_t k_stride_tok, int64_t k_stride_head,
                                  const void* v_cache, int64_t v_stride_tok, int64_t v_stride_head,
                                  const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                                  const void* b_req_idx, int req_idx_i64, const void* b_seq_len,
                                  int seq_len_i64, int64_t batch, int64_t kv_heads,
                                  int64_t head_dim, int64_t elem_bytes, int64_t max_len_in_batch,
                                  int64_t nsplit, int mode, uint32_t* sink, hipStream_t stream) {
  LL_CHECK_ARG(k_cache && v_cache && req_to_tokens && b_req_idx && b_seq_len && sink,
               "ll_probe_kv_gather: null pointer");
  const int64_t row_b = head_dim * elem_bytes;
  LL_CHECK_ARG((row_b == 128 || row_b == 256) && batch > 0 && kv_heads > 0 && nsplit > 0 &&
                   (mode == 0 || mode == 1) && max_len_in_batch > 0,
               "ll_probe_kv_gather: rows of 128 or 256 bytes, mode 0 or 1");
  GatherArgs a;
  a.k = (const char*)k_cache; a.k_st = k_stride_tok * elem_bytes; a.k_sh = k_stride_head * elem_bytes;
  a.v = (const char*)v_cache; a.v_st = v_stride_tok * elem_bytes; a.v_sh = v_stride_head * elem_bytes;
  a.r2t = req_to_tokens; a.r2t_s = req_to_tokens_stride;
  a.req_idx = b_req_idx; a.req64 = req_idx_i64;
  a.seq_len = b_seq_len; a.len64 = seq_len_i64;
  a.B = (int)batch; a.KVH = (int)kv_heads; a.nsplit = (int)nsplit;
  a.max_len = (int)max_len_in_batch; a.row_b = (int)row_b;
  a.sink = sink;
  const unsigned grid = (unsigned)(((batch + 7) / 8) * 8 * kv_heads * nsplit);
  const size_t lds = (size_t)kProbeWaves * 16 * 1024;
  if (mode == 0)
    hipLaunchKernelGGL(kv_gather_kernel<0>, dim3(grid), dim3(kProbeWaves * 64), 0, stream, a);
  else
    hipLaunchKernelGGL(kv_gather_kernel<1>, dim3(grid), dim3(kProbeWaves * 64), lds, stream, a);
  LL_RETURN_LAUNCH();
}

extern "C" int ll_probe_launch(void* dst, int64_t write_bytes, int64_t workgroups,
                               hipStream_t stream) {
  LL_CHECK_ARG(write_bytes >= 0 && write_bytes % 16 == 0 && ((uintptr_t)dst % 16) == 0 &&
                   (write_bytes == 0 || dst != nullptr),
               "ll_probe_launch: needs a 16-byte aligned buffer of 16-byte units");
  LL_CHECK_ARG(workgroups > 0 && workgroups <= (1 << 20), "ll_probe_launch: bad grid");
  hipLaunchKernelGGL(launch_probe_kernel, dim3((unsigned)workgroups), dim3(512), 0, stream,
                     (u32x4*)dst, write_bytes / 16);
  LL_RETURN_LAUNCH();
}
