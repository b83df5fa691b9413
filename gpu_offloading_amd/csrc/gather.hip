// Block-table gather: packs the scattered 16-token blocks of each sequence into
// a contiguous [tokens, num_kv_heads, head_dim] staging tensor (the closed-form
// inverse of the append: cache[bt[seq, :nb]].flatten(0, 1)[:len]).
//
// Design: grid (ceil(max_seq_len / kTokPerWG), batch).  A 256-thread workgroup
// copies kTokPerWG consecutive output rows of one sequence; the work unit is a
// 16-byte chunk of a K or V row and each lane keeps kUnroll chunks in flight.
// Cache rows are read with non-temporal loads; 8 rows per workgroup (more
// workgroups in flight) measured best.
// A token row is contiguous in both the cache and the output, and rows of the
// same block are adjacent in the cache, so loads and stores are coalesced.
// Block (swap) gather/scatter of whole blocks lives in swap.hip.
#include "kvc_common.h"

#include <algorithm>

namespace kvc {
namespace {

constexpr int kThreads = 256;
constexpr int kTokPerWG = 8;
constexpr int kUnroll = 8;

struct GatherArgs {
  const char* key_cache;
  const char* value_cache;
  const int32_t* block_table;
  int64_t bt_stride;          // elements between block-table rows
  int32_t bt_width;           // entries per block-table row
  const int32_t* cu_seq_lens;
  const int32_t* seq_starts;  // may be null
  int64_t block_stride;       // bytes
  int64_t token_stride;       // bytes
  int64_t num_blocks;
  char* out_key;
  char* out_value;
  int64_t out_stride;         // bytes between output rows
  int64_t out_rows;           // rows the outputs hold; rows past them are not written
  int32_t block_size;
  int32_t row_units;          // 16-byte chunks (or elements) per row
  int32_t* oob_count;
};

template <int kRowChunks>
__global__ __launch_bounds__(kThreads) void gather_vec16_kernel(GatherArgs a) {
  const int b = blockIdx.y;
  const int row0 = a.cu_seq_lens[b];
  const int len = a.cu_seq_lens[b + 1] - row0;
  const int i0 = blockIdx.x * kTokPerWG;
  if (i0 >= len) return;
  const int ntok = min(kTokPerWG, len - i0);
  const int start = a.seq_starts ? a.seq_starts[b] : 0;
  const uint32_t rc = kRowChunks > 0 ? uint32_t(kRowChunks) : uint32_t(a.row_units);
  const uint32_t per_tok = 2u * rc;
  const uint32_t total = uint32_t(ntok) * per_tok;
  const int32_t* bt_row = a.block_table + int64_t(b) * a.bt_stride;

  for (uint32_t base = threadIdx.x; base < total; base += kThreads * kUnroll) {
    uint4 buf[kUnroll];
    char* dst[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t item = base + uint32_t(u) * kThreads;
      dst[u] = nullptr;
      if (item >= total) continue;
      const uint32_t t = item / per_tok;
      const uint32_t rem = item - t * per_tok;
      const bool is_v = rem >= rc;
      const uint32_t chunk = is_v ? rem - rc : rem;
      const int64_t orow = int64_t(row0) + i0 + int(t);
      if (orow < 0 || orow >= a.out_rows) {
        if (a.oob_count && chunk == 0 && !is_v) atomicAdd(a.oob_count, 1);
        continue;
      }
      const int pos = start + i0 + int(t);
      const int page = pos >= 0 ? pos / a.block_size : -1;
      const int32_t blk = (page >= 0 && page < a.bt_width) ? bt_row[page] : -1;
      const int off = pos - page * a.block_size;
      dst[u] = (is_v ? a.out_value : a.out_key) + orow * a.out_stride + chunk * 16u;
      if (blk < 0 || blk >= a.num_blocks) {
        buf[u] = make_uint4(0, 0, 0, 0);
        if (a.oob_count && chunk == 0 && !is_v) atomicAdd(a.oob_count, 1);
        continue;
      }
      const char* src = (is_v ? a.value_cache : a.key_cache) +
                        int64_t(blk) * a.block_stride + int64_t(off) * a.token_stride +
                        chunk * 16u;
      buf[u] = load_stream(src);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (dst[u]) *reinterpret_cast<uint4*>(dst[u]) = buf[u];
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void gather_elem_kernel(GatherArgs a) {
  const int b = blockIdx.y;
  const int row0 = a.cu_seq_lens[b];
  const int len = a.cu_seq_lens[b + 1] - row0;
  const int i0 = blockIdx.x * kTokPerWG;
  if (i0 >= len) return;
  const int ntok = min(kTokPerWG, len - i0);
  const int start = a.seq_starts ? a.seq_starts[b] : 0;
  const uint32_t re = uint32_t(a.row_units);
  const uint32_t per_tok = 2u * re;
  const uint32_t total = uint32_t(ntok) * per_tok;
  const int32_t* bt_row = a.block_table + int64_t(b) * a.bt_stride;
  for (uint32_t item = threadIdx.x; item < total; item += kThreads) {
    const uint32_t t = item / per_tok;
    const uint32_t rem = item - t * per_tok;
    const bool is_v = rem >= re;
    const uint32_t e = is_v ? rem - re : rem;
    const int64_t orow = int64_t(row0) + i0 + int(t);
    if (orow < 0 || orow >= a.out_rows) {
      if (a.oob_count && e == 0 && !is_v) atomicAdd(a.oob_count, 1);
      continue;
    }
    const int pos = start + i0 + int(t);
    const int page = pos >= 0 ? pos / a.block_size : -1;
    const int32_t blk = (page >= 0 && page < a.bt_width) ? bt_row[page] : -1;
    const int off = pos - page * a.block_size;
    T* dst = reinterpret_cast<T*>((is_v ? a.out_value : a.out_key) + orow * a.out_stride);
    if (blk < 0 || blk >= a.num_blocks) {
      dst[e] = T(0);
      if (a.oob_count && e == 0 && !is_v) atomicAdd(a.oob_count, 1);
      continue;
    }
    const T* src = reinterpret_cast<const T*>(
        (is_v ? a.value_cache : a.key_cache) + int64_t(blk) * a.block_stride +
        int64_t(off) * a.token_stride);
    dst[e] = src[e];
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_gather_kv(
    const void* key_cache, const void* value_cache, const int32_t* block_table,
    int64_t block_table_row_stride, int32_t block_table_width,
    const int32_t* cu_seq_lens,
    const int32_t* seq_starts, int32_t batch, int32_t max_seq_len,
    int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int64_t num_blocks, int32_t elem_bytes, int64_t cache_block_stride,
    int64_t cache_token_stride, void* out_key, void* out_value,
    int64_t out_token_stride, int64_t out_rows, int32_t* oob_count, void* stream) {
  KVC_REQUIRE(batch >= 0 && max_seq_len >= 0 && out_rows >= 0, KVC_ERR_INVALID_ARG,
              "negative batch, max_seq_len or out_rows");
  if (batch == 0 || max_seq_len == 0) return ok();
  KVC_REQUIRE(key_cache && value_cache && block_table && cu_seq_lens &&
                  out_key && out_value,
              KVC_ERR_INVALID_ARG, "null pointer");
  KVC_REQUIRE(batch <= 65535, KVC_ERR_INVALID_ARG, "batch > 65535");
  KVC_REQUIRE(num_kv_heads > 0 && head_dim > 0 && block_size > 0 &&
                  num_blocks > 0 && block_table_width > 0,
              KVC_ERR_INVALID_ARG, "non-positive shape");
  KVC_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4,
              KVC_ERR_UNSUPPORTED, "elem_bytes must be 1, 2 or 4");
  const int64_t row_elems = int64_t(num_kv_heads) * head_dim;
  KVC_REQUIRE(cache_token_stride >= row_elems &&
                  cache_block_stride >= cache_token_stride * block_size &&
                  out_token_stride >= row_elems,
              KVC_ERR_INVALID_ARG, "strides smaller than a row/block");
  KVC_REQUIRE(row_elems * elem_bytes * 2 * 16 < (int64_t(1) << 31),
              KVC_ERR_INVALID_ARG, "token row too large");

  GatherArgs a;
  a.key_cache = static_cast<const char*>(key_cache);
  a.value_cache = static_cast<const char*>(value_cache);
  a.block_table = block_table;
  a.bt_stride = block_table_row_stride;
  a.bt_width = block_table_width;
  a.cu_seq_lens = cu_seq_lens;
  a.seq_starts = seq_starts;
  a.block_stride = cache_block_stride * elem_bytes;
  a.token_stride = cache_token_stride * elem_bytes;
  a.num_blocks = num_blocks;
  a.out_key = static_cast<char*>(out_key);
  a.out_value = static_cast<char*>(out_value);
  a.out_stride = out_token_stride * elem_bytes;
  a.out_rows = out_rows;
  a.block_size = block_size;
  a.oob_count = oob_count;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(unsigned(cdiv(max_seq_len, kTokPerWG)), unsigned(batch));

  const int64_t row_bytes = row_elems * elem_bytes;
  const bool vec = (row_bytes % 16 == 0) && aligned(key_cache, 16) &&
                   aligned(value_cache, 16) && aligned(out_key, 16) &&
                   aligned(out_value, 16) && a.block_stride % 16 == 0 &&
                   a.token_stride % 16 == 0 && a.out_stride % 16 == 0;
  if (vec) {
    a.row_units = int32_t(row_bytes / 16);
    if (a.row_units == 128)
      gather_vec16_kernel<128><<<grid, kThreads, 0, s>>>(a);
    else
      gather_vec16_kernel<0><<<grid, kThreads, 0, s>>>(a);
  } else {
    KVC_REQUIRE(aligned(key_cache, elem_bytes) && aligned(value_cache, elem_bytes) &&
                    aligned(out_key, elem_bytes) && aligned(out_value, elem_bytes),
                KVC_ERR_ALIGNMENT, "pointers not aligned to elem_bytes");
    a.row_units = int32_t(row_elems);
    if (elem_bytes == 2)
      gather_elem_kernel<uint16_t><<<grid, kThreads, 0, s>>>(a);
    else if (elem_bytes == 4)
      gather_elem_kernel<uint32_t><<<grid, kThreads, 0, s>>>(a);
    else
      gather_elem_kernel<uint8_t><<<grid, kThreads, 0, s>>>(a);
  }
  KVC_LAUNCH_CHECK();
  return ok();
}
