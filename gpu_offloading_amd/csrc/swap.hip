// (a10) KV block eviction / restore.
//
// The reference MoE engine has no KV swap (preemption frees and recomputes,
// src/MoE/scheduler.py:315-378); its precedents are the whole-cache
// kv_snapshot/kv_restore (src/MoE/moe_engine.py:4163-4183) and the pinned
// host buffers + side-stream H2D/D2H copies of
// src/dense/include/paged_offload_transformer.py:111-134, 394-418.  Here the
// victims are arbitrary, non-contiguous block ids, so a swap is
//   out: gather blocks -> contiguous HBM staging -> hipMemcpyAsync D2H
//   in : hipMemcpyAsync H2D -> staging -> scatter into blocks
// all on the caller's (side) stream.  A block is block_bytes contiguous bytes
// per layer for K and the same for V; staging is [n][2][block_bytes].
//
// The block copy kernels move 16-byte words: grid (chunks, n), a 256-thread
// workgroup copies kBytesPerWG bytes of one block with kUnroll loads in flight
// per lane.  The whole op is bound by the host link (PCIe), not by HBM.
#include "kvc_common.h"

#include <algorithm>

namespace kvc {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;
constexpr int64_t kBytesPerWG = int64_t(kThreads) * kUnroll * 16;  // 32 KiB

struct BlockCopyArgs {
  char* key_cache;
  char* value_cache;
  int64_t block_stride;  // bytes
  int64_t block_bytes;   // multiple of 16
  int64_t num_blocks;
  const int32_t* ids;
  char* staging;         // [n][2][block_bytes]
  int32_t* oob_count;
};

// kToStaging: cache -> staging (gather); otherwise staging -> cache (scatter).
template <bool kToStaging>
__global__ __launch_bounds__(kThreads) void block_copy_kernel(BlockCopyArgs a) {
  const int64_t i = blockIdx.y;  // position in the id list
  const int32_t id = a.ids[i];
  if (id < 0 || id >= a.num_blocks) {
    if (a.oob_count && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(a.oob_count, 1);
    return;
  }
  // Both halves (K, V) of the block: linear byte range [0, 2*block_bytes).
  const int64_t span = 2 * a.block_bytes;
  const int64_t beg = int64_t(blockIdx.x) * kBytesPerWG;
  uint4 buf[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t off = beg + (int64_t(u) * kThreads + threadIdx.x) * 16;
    if (off >= span) continue;
    const bool is_v = off >= a.block_bytes;
    const int64_t in_blk = is_v ? off - a.block_bytes : off;
    char* cache = (is_v ? a.value_cache : a.key_cache) + int64_t(id) * a.block_stride + in_blk;
    char* stage = a.staging + i * span + off;
    buf[u] = kToStaging ? load_stream(cache) : *reinterpret_cast<const uint4*>(stage);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t off = beg + (int64_t(u) * kThreads + threadIdx.x) * 16;
    if (off >= span) continue;
    const bool is_v = off >= a.block_bytes;
    const int64_t in_blk = is_v ? off - a.block_bytes : off;
    char* cache = (is_v ? a.value_cache : a.key_cache) + int64_t(id) * a.block_stride + in_blk;
    char* stage = a.staging + i * span + off;
    if (kToStaging)
      *reinterpret_cast<uint4*>(stage) = buf[u];
    else
      store_stream(cache, buf[u]);
  }
}

int check_block_args(const void* kc, const void* vc, int64_t stride,
                     int64_t block_bytes, int64_t num_blocks, const void* ids,
                     int64_t n, const void* staging) {
  KVC_REQUIRE(n >= 0, KVC_ERR_INVALID_ARG, "n < 0");
  if (n == 0) return ok();
  KVC_REQUIRE(kc && vc && ids && staging, KVC_ERR_INVALID_ARG, "null pointer");
  KVC_REQUIRE(block_bytes > 0 && block_bytes % 16 == 0, KVC_ERR_ALIGNMENT,
              "block_bytes must be a positive multiple of 16");
  KVC_REQUIRE(stride >= block_bytes && stride % 16 == 0, KVC_ERR_ALIGNMENT,
              "block stride must be >= block_bytes and a multiple of 16");
  KVC_REQUIRE(num_blocks > 0, KVC_ERR_INVALID_ARG, "num_blocks <= 0");
  KVC_REQUIRE(aligned(kc, 16) && aligned(vc, 16) && aligned(staging, 16),
              KVC_ERR_ALIGNMENT, "cache/staging pointers must be 16-byte aligned");
  return ok();
}

int launch_block_copy(bool to_staging, const void* kc, const void* vc,
                      int64_t stride, int64_t block_bytes, int64_t num_blocks,
                      const int32_t* ids, int64_t n, void* staging,
                      int32_t* oob_count, hipStream_t s) {
  BlockCopyArgs a;
  a.key_cache = const_cast<char*>(static_cast<const char*>(kc));
  a.value_cache = const_cast<char*>(static_cast<const char*>(vc));
  a.block_stride = stride;
  a.block_bytes = block_bytes;
  a.num_blocks = num_blocks;
  a.ids = ids;
  a.staging = static_cast<char*>(staging);
  a.oob_count = oob_count;
  const unsigned gx = unsigned((2 * block_bytes + kBytesPerWG - 1) / kBytesPerWG);
  constexpr int64_t kMaxY = 65535;  // grid.y limit: launch long id lists in pieces
  for (int64_t i = 0; i < n; i += kMaxY) {
    const int64_t c = std::min(kMaxY, n - i);
    a.ids = ids + i;
    a.staging = static_cast<char*>(staging) + i * 2 * block_bytes;
    const dim3 grid(gx, unsigned(c));
    if (to_staging)
      block_copy_kernel<true><<<grid, kThreads, 0, s>>>(a);
    else
      block_copy_kernel<false><<<grid, kThreads, 0, s>>>(a);
    KVC_LAUNCH_CHECK();
  }
  return ok();
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_gather_blocks(const void* key_cache, const void* value_cache,
                                 int64_t cache_block_stride_bytes, int64_t block_bytes,
                                 int64_t num_blocks, const int32_t* block_ids, int64_t n,
                                 void* staging, int32_t* oob_count, void* stream) {
  int st = check_block_args(key_cache, value_cache, cache_block_stride_bytes, block_bytes,
                            num_blocks, block_ids, n, staging);
  if (st != KVC_OK || n == 0) return st;
  return launch_block_copy(true, key_cache, value_cache, cache_block_stride_bytes,
                           block_bytes, num_blocks, block_ids, n, staging, oob_count,
                           static_cast<hipStream_t>(stream));
}

extern "C" int kvc_scatter_blocks(const void* staging, const int32_t* block_ids, int64_t n,
                                  void* key_cache, void* value_cache,
                                  int64_t cache_block_stride_bytes, int64_t block_bytes,
                                  int64_t num_blocks, int32_t* oob_count, void* stream) {
  int st = check_block_args(key_cache, value_cache, cache_block_stride_bytes, block_bytes,
                            num_blocks, block_ids, n, staging);
  if (st != KVC_OK || n == 0) return st;
  return launch_block_copy(false, key_cache, value_cache, cache_block_stride_bytes,
                           block_bytes, num_blocks, block_ids, n,
                           const_cast<void*>(staging), oob_count,
                           static_cast<hipStream_t>(stream));
}

extern "C" int kvc_swap_out(const void* key_cache, const void* value_cache,
                            int64_t cache_block_stride_bytes, int64_t block_bytes,
                            int64_t num_blocks, const int32_t* block_ids, int64_t n,
                            void* staging, int64_t staging_bytes, void* host_dst,
                            int32_t* oob_count, void* stream) {
  int st = check_block_args(key_cache, value_cache, cache_block_stride_bytes, block_bytes,
                            num_blocks, block_ids, n, staging);
  if (st != KVC_OK || n == 0) return st;
  KVC_REQUIRE(host_dst, KVC_ERR_INVALID_ARG, "null host buffer");
  const int64_t per = 2 * block_bytes;
  KVC_REQUIRE(staging_bytes >= per, KVC_ERR_WORKSPACE,
              "staging smaller than one block (" + std::to_string(per) + " bytes)");
  const int64_t chunk = staging_bytes / per;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int64_t i = 0; i < n; i += chunk) {
    const int64_t c = std::min(chunk, n - i);
    st = launch_block_copy(true, key_cache, value_cache, cache_block_stride_bytes,
                           block_bytes, num_blocks, block_ids + i, c, staging, oob_count, s);
    if (st != KVC_OK) return st;
    KVC_HIP_CHECK(hipMemcpyAsync(static_cast<char*>(host_dst) + i * per, staging, c * per,
                                 hipMemcpyDeviceToHost, s));
  }
  return ok();
}

extern "C" int kvc_swap_in(const void* host_src, const int32_t* block_ids, int64_t n,
                           void* key_cache, void* value_cache,
                           int64_t cache_block_stride_bytes, int64_t block_bytes,
                           int64_t num_blocks, void* staging, int64_t staging_bytes,
                           int32_t* oob_count, void* stream) {
  int st = check_block_args(key_cache, value_cache, cache_block_stride_bytes, block_bytes,
                            num_blocks, block_ids, n, staging);
  if (st != KVC_OK || n == 0) return st;
  KVC_REQUIRE(host_src, KVC_ERR_INVALID_ARG, "null host buffer");
  const int64_t per = 2 * block_bytes;
  KVC_REQUIRE(staging_bytes >= per, KVC_ERR_WORKSPACE,
              "staging smaller than one block (" + std::to_string(per) + " bytes)");
  const int64_t chunk = staging_bytes / per;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int64_t i = 0; i < n; i += chunk) {
    const int64_t c = std::min(chunk, n - i);
    KVC_HIP_CHECK(hipMemcpyAsync(staging, static_cast<const char*>(host_src) + i * per,
                                 c * per, hipMemcpyHostToDevice, s));
    st = launch_block_copy(false, key_cache, value_cache, cache_block_stride_bytes,
                           block_bytes, num_blocks, block_ids + i, c, staging, oob_count, s);
    if (st != KVC_OK) return st;
  }
  return ok();
}
