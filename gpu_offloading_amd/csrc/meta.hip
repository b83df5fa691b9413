// (f1) Step-setup metadata kernels.
//
// kvc_compute_slot_mapping restates, in one launch, what the reference engine
// gets from vLLM's prepare_pos_seq_lens + _compute_slot_mappings_kernel
// (src/MoE/moe_engine.py:3514-3541; eager twins :1308-1316, :2677-2695,
// continuation :1678-1695): token i of request r sits at position
// num_computed[seq] + (i - query_start_loc[r]) and goes to slot
// block_table[seq, pos // bs] * bs + pos % bs; padding tokens get slot -1.
//
// kvc_copy_page_indices restates _copy_page_indices_kernel after the row
// index_select (moe_engine.py:1937-1946): the first indptr[r+1]-indptr[r]
// entries of block-table row seq_ids[r] are flattened into indices[indptr[r]:]
// (clamped to the buffer's capacity).
//
// kvc_stage_from_host stands for the engine's pinned-buffer .copy_(...,
// non_blocking=True) uploads of the step metadata (moe_engine.py:3493-3494,
// 3506-3507): one kernel on the caller's stream reads the step's pinned int32
// image over the host link and writes it to device memory.  A hipMemcpyAsync
// of pinned memory runs on a copy engine: the compute queue then waits on it,
// and when that queue is still busy with the previous step (a replayed
// graph) the host thread issuing the copy was measured blocked for hundreds
// of microseconds.
#include "kvc_common.h"

#include <algorithm>

namespace kvc {
namespace {

struct SlotArgs {
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_rows;
  int32_t bt_width;
  const int32_t* seq_ids;
  const int32_t* qsl;
  const int32_t* num_computed;
  int32_t num_reqs;
  int32_t num_tokens;
  int32_t num_padded;
  int32_t block_size;
  int64_t* slots;
  int32_t* positions;
};

__global__ __launch_bounds__(256) void slot_mapping_kernel(SlotArgs a) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.num_padded) return;
  if (t >= a.num_tokens) {
    a.slots[t] = -1;
    if (a.positions) a.positions[t] = 0;
    return;
  }
  // Request owning token t: last r with qsl[r] <= t (binary search).
  int lo = 0, hi = a.num_reqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.qsl[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int r = lo;
  const int seq = a.seq_ids[r];
  if (seq < 0 || seq >= a.bt_rows) {
    a.slots[t] = -1;
    if (a.positions) a.positions[t] = 0;
    return;
  }
  const int pos = a.num_computed[seq] + (t - a.qsl[r]);
  const int page = pos / a.block_size;
  int64_t slot = -1;
  if (pos >= 0 && page < a.bt_width) {
    const int32_t blk = a.bt[int64_t(seq) * a.bt_stride + page];
    slot = int64_t(blk) * a.block_size + (pos - page * a.block_size);
  }
  a.slots[t] = slot;
  if (a.positions) a.positions[t] = pos;
}

__global__ __launch_bounds__(256) void copy_page_indices_kernel(
    const int32_t* bt, int64_t bt_stride, int32_t rows, const int32_t* seq_ids,
    const int32_t* indptr, int32_t width, int32_t* indices, int64_t capacity) {
  const int r = blockIdx.x;
  const int row = seq_ids ? seq_ids[r] : r;
  if (row < 0 || row >= rows) return;
  const int beg = indptr[r];
  if (beg < 0) return;
  // Entries past the indices buffer (an indptr larger than the buffer) are
  // not written.
  const int n = int(min<int64_t>(min(indptr[r + 1] - beg, width), capacity - beg));
  const int32_t* src = bt + int64_t(row) * bt_stride;
  for (int j = threadIdx.x; j < n; j += 256) indices[beg + j] = src[j];
}

// Four int32 per thread: ranges [0, head) and [tail_begin, tail_end) of the
// image, tail_begin a multiple of 4, both buffers 16-byte aligned.  The host
// loads are system-scope, so they read memory, not a cached older image.
__global__ __launch_bounds__(256) void stage_kernel(const int32_t* __restrict__ host,
                                                    int32_t* __restrict__ dev, int64_t head,
                                                    int64_t tail_begin, int64_t tail_end) {
  int64_t q = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t head_quads = (head + 3) >> 2;
  int64_t beg, end;
  if (q < head_quads) {
    beg = q << 2;
    end = min(beg + 4, head);
  } else {
    beg = tail_begin + ((q - head_quads) << 2);
    if (beg >= tail_end) return;
    end = min(beg + 4, tail_end);
  }
  if (end - beg == 4) {
    const uint64_t* s = reinterpret_cast<const uint64_t*>(host + beg);
    const uint64_t lo = __hip_atomic_load(s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const uint64_t hi = __hip_atomic_load(s + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    *reinterpret_cast<uint4*>(dev + beg) =
        make_uint4(uint32_t(lo), uint32_t(lo >> 32), uint32_t(hi), uint32_t(hi >> 32));
  } else {
    for (int64_t i = beg; i < end; ++i)
      dev[i] = __hip_atomic_load(host + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_stage_from_host(const int32_t* host, int32_t* dev, int64_t head,
                                   int64_t tail_begin, int64_t tail_end, void* stream) {
  KVC_REQUIRE(head >= 0 && tail_begin >= head && tail_end >= tail_begin,
              KVC_ERR_INVALID_ARG, "need 0 <= head <= tail_begin <= tail_end");
  KVC_REQUIRE((tail_begin & 3) == 0, KVC_ERR_INVALID_ARG, "tail_begin must be a multiple of 4");
  const int64_t quads = ((head + 3) >> 2) + ((tail_end - tail_begin + 3) >> 2);
  if (quads == 0) return ok();
  KVC_REQUIRE(host && dev, KVC_ERR_INVALID_ARG, "null pointer");
  KVC_REQUIRE((reinterpret_cast<uintptr_t>(host) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(dev) & 15) == 0,
              KVC_ERR_INVALID_ARG, "host and dev must be 16-byte aligned");
  // The image must be pinned host memory the device can read; the kernel
  // uses the device's address of it.
  hipPointerAttribute_t attr{};
  const hipError_t e = hipPointerGetAttributes(&attr, host);
  if (e != hipSuccess) (void)hipGetLastError();  // not sticky: clear it for later checks
  KVC_REQUIRE(e == hipSuccess && attr.type == hipMemoryTypeHost && attr.devicePointer,
              KVC_ERR_INVALID_ARG, "host image is not pinned host memory (hipHostMalloc)");
  stage_kernel<<<dim3(unsigned(cdiv(quads, 256))), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const int32_t*>(attr.devicePointer), dev, head, tail_begin, tail_end);
  KVC_LAUNCH_CHECK();
  return ok();
}

extern "C" int kvc_compute_slot_mapping(
    const int32_t* block_table, int64_t block_table_row_stride, int32_t block_table_rows,
    int32_t max_pages_per_seq,
    const int32_t* seq_ids, const int32_t* query_start_loc, const int32_t* num_computed,
    int32_t num_reqs, int32_t num_tokens, int32_t num_tokens_padded, int32_t block_size,
    int64_t* slot_mapping, int32_t* positions, void* stream) {
  KVC_REQUIRE(num_reqs >= 0 && num_tokens >= 0 && num_tokens_padded >= num_tokens,
              KVC_ERR_INVALID_ARG, "bad counts (need num_tokens_padded >= num_tokens >= 0)");
  if (num_tokens_padded == 0) return ok();
  KVC_REQUIRE(slot_mapping, KVC_ERR_INVALID_ARG, "null slot_mapping");
  KVC_REQUIRE(num_tokens == 0 || (num_reqs > 0 && block_table && seq_ids &&
                                  query_start_loc && num_computed),
              KVC_ERR_INVALID_ARG, "null metadata pointer");
  KVC_REQUIRE(block_size > 0 && max_pages_per_seq > 0 && block_table_rows > 0,
              KVC_ERR_INVALID_ARG, "non-positive block_size / block-table shape");
  SlotArgs a{block_table, block_table_row_stride, block_table_rows, max_pages_per_seq, seq_ids,
             query_start_loc, num_computed, num_reqs, num_tokens, num_tokens_padded,
             block_size, slot_mapping, positions};
  slot_mapping_kernel<<<dim3(unsigned(cdiv(num_tokens_padded, 256))), 256, 0,
                        static_cast<hipStream_t>(stream)>>>(a);
  KVC_LAUNCH_CHECK();
  return ok();
}

extern "C" int kvc_copy_page_indices(const int32_t* block_table,
                                     int64_t block_table_row_stride,
                                     int32_t block_table_rows,
                                     const int32_t* seq_ids, const int32_t* indptr,
                                     int32_t num_reqs, int32_t max_pages_per_req,
                                     int32_t* indices, int64_t indices_capacity,
                                     void* stream) {
  KVC_REQUIRE(num_reqs >= 0 && indices_capacity >= 0, KVC_ERR_INVALID_ARG,
              "num_reqs or indices_capacity < 0");
  if (num_reqs == 0) return ok();
  KVC_REQUIRE(block_table && indptr && indices, KVC_ERR_INVALID_ARG, "null pointer");
  KVC_REQUIRE(block_table_rows > 0 && max_pages_per_req > 0, KVC_ERR_INVALID_ARG,
              "non-positive block-table shape");
  copy_page_indices_kernel<<<dim3(unsigned(num_reqs)), 256, 0,
                             static_cast<hipStream_t>(stream)>>>(
      block_table, block_table_row_stride, block_table_rows, seq_ids, indptr,
      max_pages_per_req, indices, indices_capacity);
  KVC_LAUNCH_CHECK();
  return ok();
}
