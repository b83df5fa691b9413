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

// One-launch setup of a pure-decode step.  Workgroup w streams requests
// 4w .. 4w+3 (one wave each) and every workgroup copies its share of the image
// to the device and of the new lengths.  All step fields are read straight
// from the pinned image (system-scope loads), so no workgroup waits for
// another: every workgroup applies all of the step's block-table writes
// itself (the same values at the same places, so the repeats are harmless)
// before its barrier, and then reads only rows of its own requests.
constexpr int kSetupWaves = 4;

struct StepSetupArgs {
  const int32_t* host;     // the pinned image, device-visible address
  int32_t* dev;            // its device copy
  int64_t head, tail_begin, tail_end;
  int64_t o_ids, o_pos, o_indptr, o_lens, o_bt_pos, o_bt_val;
  int32_t num_reqs, num_writes, max_seqs, block_size;
  int32_t* bt;
  int64_t bt_stride;
  int32_t bt_rows, bt_width;
  int32_t* seq_lens;
  int64_t* slots;
  int32_t num_slots;
  int32_t* indices;
  int64_t capacity;
};

__device__ __forceinline__ int32_t host_i32(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ __launch_bounds__(64 * kSetupWaves) void decode_step_setup_kernel(StepSetupArgs a) {
  const int tid = threadIdx.x;
  const int64_t gtid = int64_t(blockIdx.x) * blockDim.x + tid;
  const int64_t gthreads = int64_t(gridDim.x) * blockDim.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r = blockIdx.x * kSetupWaves + wave;
  const bool live = r < a.num_reqs;  // wave-uniform
  // The request's fields first (one load round trip over the host link).
  int32_t seq = -1, pos = -1, beg = 0, end = 0;
  if (live) {
    seq = host_i32(a.host + a.o_ids + r);
    pos = host_i32(a.host + a.o_pos + r);
    beg = host_i32(a.host + a.o_indptr + r);
    end = host_i32(a.host + a.o_indptr + r + 1);
  }
  // Every load over the host link of a thread's first pass is issued before
  // any store that needs one, so the kernel waits for the link about once;
  // the loops after them only run for images larger than the grid.
  // The step's block-table writes (flat position = row * width + column).
  constexpr int kWrites = 4;
  int64_t wp[kWrites];
  int32_t wv[kWrites];
#pragma unroll
  for (int i = 0; i < kWrites; ++i) {
    const int k = tid + i * int(blockDim.x);
    wp[i] = -1;
    wv[i] = 0;
    if (k < a.num_writes) {
      wp[i] = __hip_atomic_load(reinterpret_cast<const int64_t*>(a.host + a.o_bt_pos) + k,
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      wv[i] = host_i32(a.host + a.o_bt_val + k);
    }
  }
  // The device lengths after the step.
  const bool has_len = gtid < a.max_seqs;
  const int32_t len0 = has_len ? host_i32(a.host + a.o_lens + gtid) : 0;
  // The image's device copy: one 16-byte quad per thread and pass, as two
  // 8-byte loads where the quad lies inside a range.
  const int64_t head_quads = (a.head + 3) >> 2;
  const int64_t quads = head_quads + ((a.tail_end - a.tail_begin + 3) >> 2);
  auto quad_range = [&](int64_t q, int64_t& b0, int64_t& b1) __attribute__((always_inline)) {
    if (q < head_quads) {
      b0 = q << 2;
      b1 = min(b0 + 4, a.head);
    } else {
      b0 = a.tail_begin + ((q - head_quads) << 2);
      b1 = min(b0 + 4, a.tail_end);
    }
  };
  auto load_quad = [&](int64_t b0, int64_t b1, int32_t (&v)[4]) __attribute__((always_inline)) {
    if (b1 - b0 == 4) {
      const uint64_t* src = reinterpret_cast<const uint64_t*>(a.host + b0);
      const uint64_t lo = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      const uint64_t hi = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      v[0] = int32_t(lo);
      v[1] = int32_t(lo >> 32);
      v[2] = int32_t(hi);
      v[3] = int32_t(hi >> 32);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = b0 + i < b1 ? host_i32(a.host + b0 + i) : 0;
    }
  };
  auto store_quad = [&](int64_t b0, int64_t b1, const int32_t (&v)[4]) __attribute__((always_inline)) {
    if (b1 - b0 == 4) {
      *reinterpret_cast<int4*>(a.dev + b0) = make_int4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (b0 + i < b1) a.dev[b0 + i] = v[i];
    }
  };
  int64_t qb0 = 0, qb1 = 0;
  int32_t qv[4] = {0, 0, 0, 0};
  if (gtid < quads) {
    quad_range(gtid, qb0, qb1);
    load_quad(qb0, qb1, qv);
  }
  // Stores.
  if (gtid < quads) store_quad(qb0, qb1, qv);
  if (has_len) a.seq_lens[gtid] = len0;
  for (int64_t t = a.num_reqs + gtid; t < a.num_slots; t += gthreads) a.slots[t] = -1;
  const int64_t cells = int64_t(a.bt_rows) * a.bt_width;
#pragma unroll
  for (int i = 0; i < kWrites; ++i) {
    if (wp[i] >= 0 && wp[i] < cells) {
      const int64_t row = wp[i] / a.bt_width;
      a.bt[row * a.bt_stride + (wp[i] - row * a.bt_width)] = wv[i];
    }
  }
  // Larger images, lengths and write lists.
  for (int64_t q = gtid + gthreads; q < quads; q += gthreads) {
    int64_t b0, b1;
    int32_t v[4];
    quad_range(q, b0, b1);
    load_quad(b0, b1, v);
    store_quad(b0, b1, v);
  }
  for (int64_t i = gtid + gthreads; i < a.max_seqs; i += gthreads)
    a.seq_lens[i] = host_i32(a.host + a.o_lens + i);
  for (int k = tid + kWrites * int(blockDim.x); k < a.num_writes; k += blockDim.x) {
    const int64_t p = __hip_atomic_load(reinterpret_cast<const int64_t*>(a.host + a.o_bt_pos) + k,
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int32_t v = host_i32(a.host + a.o_bt_val + k);
    if (p >= 0 && p < cells) {
      const int64_t row = p / a.bt_width;
      a.bt[row * a.bt_stride + (p - row * a.bt_width)] = v;
    }
  }
  __syncthreads();  // this workgroup's block-table writes are visible to it
  if (!live || seq < 0 || seq >= a.bt_rows) {
    if (live && lane == 0) a.slots[r] = -1;
    return;
  }
  const int32_t* row = a.bt + int64_t(seq) * a.bt_stride;
  if (lane == 0) {
    const int page = pos / a.block_size;
    int64_t slot = -1;
    if (pos >= 0 && page < a.bt_width)
      slot = int64_t(row[page]) * a.block_size + (pos - page * a.block_size);
    a.slots[r] = slot;
  }
  // Page-index flatten: four loads in flight per lane before their stores.
  if (beg < 0) return;
  const int n = int(min<int64_t>(min(end - beg, a.bt_width), a.capacity - beg));
  for (int j0 = 0; j0 < n; j0 += 256) {
    int32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = j0 + 64 * i + lane;
      v[i] = j < n ? row[j] : 0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = j0 + 64 * i + lane;
      if (j < n) a.indices[beg + j] = v[i];
    }
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_decode_step_setup(const int32_t* host_image, int32_t* dev_image,
                                     const kvc_decode_step_layout* layout,
                                     int32_t* block_table, int64_t block_table_row_stride,
                                     int32_t block_table_rows, int32_t max_pages_per_seq,
                                     int32_t* seq_lens, int64_t* slot_mapping,
                                     int32_t num_slots, int32_t* indices,
                                     int64_t indices_capacity, void* stream) {
  KVC_REQUIRE(layout, KVC_ERR_INVALID_ARG, "null layout");
  const kvc_decode_step_layout& L = *layout;
  KVC_REQUIRE(L.num_reqs >= 0 && L.num_bt_writes >= 0 && L.max_seqs >= 0 &&
                  L.block_size > 0 && num_slots >= L.num_reqs && indices_capacity >= 0,
              KVC_ERR_INVALID_ARG, "bad counts (need num_slots >= num_reqs >= 0)");
  KVC_REQUIRE(L.plan_ints >= 0 && L.tail_begin >= L.plan_ints && (L.tail_begin & 3) == 0 &&
                  L.tail_end >= L.tail_begin,
              KVC_ERR_INVALID_ARG, "need 0 <= plan_ints <= tail_begin <= tail_end, "
                                   "tail_begin a multiple of 4");
  auto inside = [&](int64_t off, int64_t n) {
    return off >= L.tail_begin && off + n <= L.tail_end;
  };
  KVC_REQUIRE(inside(L.ids, L.num_reqs) && inside(L.positions, L.num_reqs) &&
                  inside(L.indptr, int64_t(L.num_reqs) + 1) &&
                  inside(L.lens_after, L.max_seqs) &&
                  inside(L.bt_pos, 2 * int64_t(L.num_bt_writes)) && (L.bt_pos & 1) == 0 &&
                  inside(L.bt_val, L.num_bt_writes),
              KVC_ERR_INVALID_ARG, "a step field lies outside the image's tail range "
                                   "(or the block-table positions are not 8-byte aligned)");
  KVC_REQUIRE(host_image && dev_image && block_table && seq_lens && slot_mapping &&
                  (indices || L.num_reqs == 0),
              KVC_ERR_INVALID_ARG, "null pointer");
  KVC_REQUIRE(block_table_rows > 0 && max_pages_per_seq > 0 &&
                  block_table_row_stride >= max_pages_per_seq,
              KVC_ERR_INVALID_ARG, "bad block-table shape");
  KVC_REQUIRE((reinterpret_cast<uintptr_t>(host_image) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(dev_image) & 15) == 0,
              KVC_ERR_ALIGNMENT, "host and dev images must be 16-byte aligned");
  hipPointerAttribute_t attr{};
  const hipError_t e = hipPointerGetAttributes(&attr, host_image);
  if (e != hipSuccess) (void)hipGetLastError();  // not sticky: clear it for later checks
  KVC_REQUIRE(e == hipSuccess && attr.type == hipMemoryTypeHost && attr.devicePointer,
              KVC_ERR_INVALID_ARG, "host image is not pinned host memory (hipHostMalloc)");
  StepSetupArgs a;
  a.host = static_cast<const int32_t*>(attr.devicePointer);
  a.dev = dev_image;
  a.head = L.plan_ints;
  a.tail_begin = L.tail_begin;
  a.tail_end = L.tail_end;
  a.o_ids = L.ids;
  a.o_pos = L.positions;
  a.o_indptr = L.indptr;
  a.o_lens = L.lens_after;
  a.o_bt_pos = L.bt_pos;
  a.o_bt_val = L.bt_val;
  a.num_reqs = L.num_reqs;
  a.num_writes = L.num_bt_writes;
  a.max_seqs = L.max_seqs;
  a.block_size = L.block_size;
  a.bt = block_table;
  a.bt_stride = block_table_row_stride;
  a.bt_rows = block_table_rows;
  a.bt_width = max_pages_per_seq;
  a.seq_lens = seq_lens;
  a.slots = slot_mapping;
  a.num_slots = num_slots;
  a.indices = indices;
  a.capacity = indices_capacity;
  const int64_t groups = std::max<int64_t>(1, cdiv(int64_t(L.num_reqs), kSetupWaves));
  KVC_REQUIRE(groups <= 65535, KVC_ERR_INVALID_ARG, "too many requests");
  decode_step_setup_kernel<<<dim3(unsigned(groups)), 64 * kSetupWaves, 0,
                             static_cast<hipStream_t>(stream)>>>(a);
  KVC_LAUNCH_CHECK();
  return ok();
}

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
