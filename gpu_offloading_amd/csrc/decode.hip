// (a6/a7/a8) Paged GQA decode attention for gfx950.
//
// Semantics: FlashInfer BatchDecodeWithPagedKVCacheWrapper.run as the reference
// engine calls it (src/MoE/moe_engine.py:3907-3909, planned at :1949-1955 with
// pos_encoding_mode="NONE", default sm_scale = 1/sqrt(head_dim)): for request b
// and query head hq, attention over the tokens held in pages
// indices[indptr[b] .. indptr[b+1]) (final page: last_page_len[b] tokens) of KV
// head hq / group.  Split-K partials are merged with the log-sum-exp rule of
// src/dense/offload_kv_attn.py:24-39 (done in base 2 here).
//
// Decode is a GEMV: every K/V byte is used by `group` query heads only, so the
// kernel is HBM-bound and runs on the VALU (no MFMA):
//   * grid (max_partitions, num_kv_heads, batch); a 256-thread workgroup owns
//     one (request, KV head, partition of pages_per_partition pages) and serves
//     all `group` query heads of that KV head, so K/V are read exactly once;
//   * each wave streams every 4th page of the partition.  A page holds 16 token
//     rows of 256 B per KV head (head_dim 128, bf16); lane (row r, column c)
//     loads 16 B (dims 8c..8c+7) of tokens r, r+4, r+8, r+12 for K and for V,
//     i.e. eight global_load_dwordx4 per lane per page, fully coalesced in 256 B
//     runs.  The next page is prefetched into a second register set while the
//     current one is consumed;
//   * q.k uses v_dot2c_f32_bf16 on the raw bf16 pairs (exact products, fp32
//     sum); the 16 lanes of a DPP row are reduced with quad_perm/row_ror DPP
//     adds; each row keeps its own online-softmax state (m, l, acc) in base 2;
//   * epilogue: rows merge with lane shuffles, the four waves merge through
//     LDS, and the workgroup writes either the final bf16 output (single
//     partition) or an fp32 partial + its log2-sum-exp to the workspace, which
//     decode_merge_kernel folds.
#include "kvc_common.h"

#include <algorithm>
#include <cmath>

namespace kvc {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPage = 16;      // tokens per page (the engine's page_size)
constexpr int kTokPerRow = 4;  // tokens of a page handled by one 16-lane row
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_stride;        // elements between requests
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t block_stride;    // elements between cache blocks
  int64_t token_stride;    // elements between tokens of a block
  int64_t num_blocks;
  const int32_t* indptr;
  const int32_t* indices;
  int64_t num_indices;
  const int32_t* last_page_len;
  float scale_log2;        // sm_scale * log2(e)
  int32_t num_kv_heads;
  int32_t pages_per_part;
  int32_t max_parts;
  float* part_o;           // [batch][Hkv][max_parts][G][D]
  float* part_lse;         // [batch][Hkv][max_parts][G]   (log2 domain)
  uint16_t* out;
  int64_t out_stride;      // elements between requests
  float* lse;              // [batch][Hq] natural log, may be null
};

// Load the D/16 bf16 elements one lane owns (D/32 32-bit words).
template <int D>
__device__ __forceinline__ void load_slice(uint32_t (&w)[D / 32],
                                           const uint16_t* p) {
  if constexpr (D == 64) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    w[0] = t.x; w[1] = t.y;
  } else if constexpr (D == 128) {
    const uint4 t = *reinterpret_cast<const uint4*>(p);
    w[0] = t.x; w[1] = t.y; w[2] = t.z; w[3] = t.w;
  } else {
    static_assert(D == 256, "head_dim must be 64, 128 or 256");
    const uint4 t0 = reinterpret_cast<const uint4*>(p)[0];
    const uint4 t1 = reinterpret_cast<const uint4*>(p)[1];
    w[0] = t0.x; w[1] = t0.y; w[2] = t0.z; w[3] = t0.w;
    w[4] = t1.x; w[5] = t1.y; w[6] = t1.z; w[7] = t1.w;
  }
}

template <int D>
struct PageRegs {
  uint32_t k[kTokPerRow][D / 32];
  uint32_t v[kTokPerRow][D / 32];
};

// Issue the loads of page `pi` (index into this request's page list) and
// return its number of valid tokens (0 for an out-of-range block id).
template <int D>
__device__ __forceinline__ int load_page(const DecodeArgs& a, PageRegs<D>& r,
                                         int64_t page_slot, int valid_tokens,
                                         int64_t lane_off) {
  int32_t blk = page_slot < a.num_indices ? a.indices[page_slot] : -1;
  if (blk < 0 || blk >= a.num_blocks) {
#pragma unroll
    for (int j = 0; j < kTokPerRow; ++j)
#pragma unroll
      for (int w = 0; w < D / 32; ++w) r.k[j][w] = r.v[j][w] = 0u;
    return 0;
  }
  const int64_t base = int64_t(blk) * a.block_stride + lane_off;
  const uint16_t* kp = a.k_cache + base;
  const uint16_t* vp = a.v_cache + base;
#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j)
    load_slice<D>(r.k[j], kp + int64_t(j) * kTokPerRow * a.token_stride);
#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j)
    load_slice<D>(r.v[j], vp + int64_t(j) * kTokPerRow * a.token_stride);
  return valid_tokens;
}

// Fold one page into the row's online-softmax state.
template <int G, int D>
__device__ __forceinline__ void consume_page(const uint32_t (&qw)[G][D / 32],
                                             PageRegs<D>& r, int valid, int row,
                                             float scale_log2, float (&m)[G],
                                             float (&l)[G],
                                             float (&acc)[G][D / 16]) {
  constexpr int W = D / 32;
  bool ok[kTokPerRow];
#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j) ok[j] = row + kTokPerRow * j < valid;
  if (valid < kPage) {
    // Stale slots past the sequence end may hold anything (even NaN bits):
    // clear their V so that 0 * v stays 0.
#pragma unroll
    for (int j = 0; j < kTokPerRow; ++j)
      if (!ok[j])
#pragma unroll
        for (int w = 0; w < W; ++w) r.v[j][w] = 0u;
  }

  float s[kTokPerRow][G];
#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) d = dot2_bf16(qw[g][w], r.k[j][w], d);
      s[j][g] = row16_sum(d) * scale_log2;
    }

  float p[kTokPerRow][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = kNegBig;
#pragma unroll
    for (int j = 0; j < kTokPerRow; ++j) mx = ok[j] ? fmaxf(mx, s[j][g]) : mx;
    const float m_new = fmaxf(m[g], mx);
    const float alpha = fast_exp2(m[g] - m_new);
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < kTokPerRow; ++j) {
      p[j][g] = ok[j] ? fast_exp2(s[j][g] - m_new) : 0.f;
      psum += p[j][g];
    }
    l[g] = l[g] * alpha + psum;
    m[g] = m_new;
#pragma unroll
    for (int e = 0; e < D / 16; ++e) acc[g][e] *= alpha;
  }

#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j)
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float v0 = bf16lo(r.v[j][w]);
      const float v1 = bf16hi(r.v[j][w]);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        acc[g][2 * w] = fmaf(p[j][g], v0, acc[g][2 * w]);
        acc[g][2 * w + 1] = fmaf(p[j][g], v1, acc[g][2 * w + 1]);
      }
    }
}

template <int G, int D>
__global__ __launch_bounds__(kThreads) void decode_partition_kernel(DecodeArgs a) {
  constexpr int W = D / 32;
  constexpr int E = D / 16;
  const int part = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int pbeg = a.indptr[b];
  const int npages = a.indptr[b + 1] - pbeg;
  const int p0 = part * a.pages_per_part;
  if (p0 >= npages) return;  // uniform over the workgroup
  const int p1 = min(p0 + a.pages_per_part, npages);
  const int nparts = (npages + a.pages_per_part - 1) / a.pages_per_part;
  const int last_len = min(max(a.last_page_len[b], 0), kPage);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int row = lane >> 4;
  const int col = lane & 15;

  uint32_t qw[G][W];
  const uint16_t* qb = a.q + int64_t(b) * a.q_stride + int64_t(h) * G * D + col * E;
#pragma unroll
  for (int g = 0; g < G; ++g) load_slice<D>(qw[g], qb + g * D);

  float m[G], l[G], acc[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
  }

  const int64_t lane_off = int64_t(row) * a.token_stride + int64_t(h) * D + col * E;
  auto valid_of = [&](int pi) { return pi == npages - 1 ? last_len : kPage; };

  // Two register sets: page pi is consumed while page pi+kWaves is in flight.
  PageRegs<D> ra, rb;
  int pi = p0 + wave;
  int va = 0, vb = 0;
  if (pi < p1) va = load_page<D>(a, ra, int64_t(pbeg) + pi, valid_of(pi), lane_off);
  while (pi < p1) {
    const int pn = pi + kWaves;
    if (pn < p1) vb = load_page<D>(a, rb, int64_t(pbeg) + pn, valid_of(pn), lane_off);
    consume_page<G, D>(qw, ra, va, row, a.scale_log2, m, l, acc);
    pi = pn;
    if (pi >= p1) break;
    const int pn2 = pi + kWaves;
    if (pn2 < p1) va = load_page<D>(a, ra, int64_t(pbeg) + pn2, valid_of(pn2), lane_off);
    consume_page<G, D>(qw, rb, vb, row, a.scale_log2, m, l, acc);
    pi = pn2;
  }

  // Merge the four rows of the wave (lanes c, c+16, c+32, c+48 hold the same dims).
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off);
      const float lo = __shfl_xor(l[g], off);
      const float mm = fmaxf(m[g], mo);
      const float wa = fast_exp2(m[g] - mm);
      const float wb = fast_exp2(mo - mm);
      l[g] = l[g] * wa + lo * wb;
      m[g] = mm;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float ao = __shfl_xor(acc[g][e], off);
        acc[g][e] = acc[g][e] * wa + ao * wb;
      }
    }
  }

  // Merge the waves through LDS.
  __shared__ float s_acc[kWaves][G][D];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < E; ++e) s_acc[wave][g][col * E + e] = acc[g][e];
      if (col == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  const int hq0 = h * G;
  const int64_t part_base = (int64_t(b) * a.num_kv_heads + h) * a.max_parts + part;
  for (int o = tid; o < G * D; o += kThreads) {
    const int g = o / D;
    const int d = o - g * D;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, s_m[w][g]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(s_m[w][g] - mm);
      L = fmaf(s_l[w][g], f, L);
      A = fmaf(s_acc[w][g][d], f, A);
    }
    const float res = L > 0.f ? A / L : 0.f;
    const float lse2 = L > 0.f ? mm + fast_log2(L) : -INFINITY;
    if (nparts == 1) {
      a.out[int64_t(b) * a.out_stride + int64_t(hq0 + g) * D + d] = f32_to_bf16(res);
      if (a.lse && d == 0)
        a.lse[int64_t(b) * a.num_kv_heads * G + hq0 + g] = lse2 * kLn2;
    } else {
      a.part_o[(part_base * G + g) * D + d] = res;
      if (d == 0) a.part_lse[part_base * G + g] = lse2;
    }
  }
}

struct MergeArgs {
  const float* part_o;
  const float* part_lse;
  const int32_t* indptr;
  int32_t pages_per_part;
  int32_t max_parts;
  int32_t num_kv_heads;
  int32_t group;
  uint16_t* out;
  int64_t out_stride;
  float* lse;
};

// Fold the partition partials of one (request, query head).  Requests with a
// single partition were finished by the partition kernel; requests with no
// pages get a zero output and lse = -inf.
template <int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(MergeArgs a) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int G = a.group;
  const int npages = a.indptr[b + 1] - a.indptr[b];
  const int nparts = min(max((npages + a.pages_per_part - 1) / a.pages_per_part, 0),
                         a.max_parts);
  if (nparts == 1) return;
  uint16_t* out = a.out + int64_t(b) * a.out_stride + int64_t(hq) * D;
  const int Hq = a.num_kv_heads * G;
  const int h = hq / G;
  const int g = hq - h * G;
  const int64_t base = (int64_t(b) * a.num_kv_heads + h) * a.max_parts;
  float mm = -INFINITY;
  for (int p = 0; p < nparts; ++p) mm = fmaxf(mm, a.part_lse[(base + p) * G + g]);
  if (nparts == 0 || mm == -INFINITY) {
    for (int d = threadIdx.x; d < D; d += 64) out[d] = 0;
    if (a.lse && threadIdx.x == 0) a.lse[int64_t(b) * Hq + hq] = -INFINITY;
    return;
  }
  float S = 0.f;
  for (int p = 0; p < nparts; ++p) S += fast_exp2(a.part_lse[(base + p) * G + g] - mm);
  const float inv = 1.f / S;
  for (int d = threadIdx.x; d < D; d += 64) {
    float acc = 0.f;
    for (int p = 0; p < nparts; ++p) {
      const float w = fast_exp2(a.part_lse[(base + p) * G + g] - mm);
      acc = fmaf(w, a.part_o[((base + p) * G + g) * D + d], acc);
    }
    out[d] = f32_to_bf16(acc * inv);
  }
  if (a.lse && threadIdx.x == 0)
    a.lse[int64_t(b) * Hq + hq] = (mm + fast_log2(S)) * kLn2;
}

template <int G, int D>
void launch_partition(const DecodeArgs& a, int batch, hipStream_t s) {
  const dim3 grid(unsigned(a.max_parts), unsigned(a.num_kv_heads), unsigned(batch));
  decode_partition_kernel<G, D><<<grid, kThreads, 0, s>>>(a);
}

template <int D>
bool dispatch_group(int group, const DecodeArgs& a, int batch, hipStream_t s) {
  switch (group) {
    case 1: launch_partition<1, D>(a, batch, s); return true;
    case 2: launch_partition<2, D>(a, batch, s); return true;
    case 4: launch_partition<4, D>(a, batch, s); return true;
    case 8: launch_partition<8, D>(a, batch, s); return true;
    default: return false;
  }
}

// Merge of two bf16 attention states (a8 as a standalone op).
__global__ __launch_bounds__(256) void merge_states_kernel(
    const uint16_t* o1, const float* lse1, const uint16_t* o2,
    const float* lse2, int64_t n, int head_dim, uint16_t* out, float* lse) {
  const int64_t total = n * head_dim;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / head_dim;
    const float l1 = lse1[r], l2 = lse2[r];
    const float mx = fmaxf(l1, l2);
    float w1, w2, nl;
    if (mx == -INFINITY) {
      w1 = w2 = 0.f;
      nl = -INFINITY;
    } else {
      const float e1 = expf(l1 - mx), e2 = expf(l2 - mx);
      nl = mx + logf(e1 + e2);
      w1 = e1 / (e1 + e2);
      w2 = e2 / (e1 + e2);
    }
    const float a1 = __uint_as_float(uint32_t(o1[i]) << 16);
    const float a2 = __uint_as_float(uint32_t(o2[i]) << 16);
    // Element i is read and written by the same thread, so out may alias o1
    // or o2; lse may not alias lse1/lse2 (checked on the host).
    out[i] = f32_to_bf16(a1 * w1 + a2 * w2);
    if (lse && i - r * head_dim == 0) lse[r] = nl;
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int64_t kvc_decode_workspace_bytes(int32_t batch, int32_t num_qo_heads,
                                              int32_t head_dim,
                                              int32_t max_partitions) {
  if (batch <= 0 || num_qo_heads <= 0 || head_dim <= 0 || max_partitions <= 1)
    return 0;
  const int64_t rows = int64_t(batch) * num_qo_heads * max_partitions;
  const int64_t o_bytes = (rows * head_dim * 4 + 255) / 256 * 256;
  const int64_t l_bytes = (rows * 4 + 255) / 256 * 256;
  return o_bytes + l_bytes;
}

extern "C" int kvc_decode_plan(const int32_t* indptr_host, int32_t batch,
                               int32_t num_qo_heads, int32_t num_kv_heads,
                               int32_t head_dim, int32_t page_size,
                               int32_t pages_per_partition_hint, int32_t num_cus,
                               kvc_decode_schedule* sched) {
  KVC_REQUIRE(sched, KVC_ERR_INVALID_ARG, "null schedule");
  KVC_REQUIRE(batch >= 0 && batch <= 65535, KVC_ERR_INVALID_ARG,
              "batch must be in [0, 65535]");
  KVC_REQUIRE(batch == 0 || indptr_host, KVC_ERR_INVALID_ARG, "null indptr");
  KVC_REQUIRE(num_qo_heads > 0 && num_kv_heads > 0 &&
                  num_qo_heads % num_kv_heads == 0,
              KVC_ERR_INVALID_ARG, "num_qo_heads must be a multiple of num_kv_heads");
  const int group = num_qo_heads / num_kv_heads;
  KVC_REQUIRE(group == 1 || group == 2 || group == 4 || group == 8,
              KVC_ERR_UNSUPPORTED, "group size must be 1, 2, 4 or 8");
  KVC_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
              KVC_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  KVC_REQUIRE(page_size == kPage, KVC_ERR_UNSUPPORTED, "page_size must be 16");
  KVC_REQUIRE(num_kv_heads <= 65535, KVC_ERR_INVALID_ARG, "too many KV heads");

  int64_t total = 0;
  int32_t max_pages = 0;
  int32_t num_empty = 0;
  for (int b = 0; b < batch; ++b) {
    const int32_t n = indptr_host[b + 1] - indptr_host[b];
    KVC_REQUIRE(n >= 0, KVC_ERR_INVALID_ARG, "indptr must be non-decreasing");
    total += n;
    max_pages = std::max(max_pages, n);
    num_empty += n == 0;
  }
  KVC_REQUIRE(batch == 0 || indptr_host[0] == 0, KVC_ERR_INVALID_ARG,
              "indptr[0] must be 0");

  int ppp;
  if (pages_per_partition_hint > 0) {
    ppp = (pages_per_partition_hint + 3) / 4 * 4;
  } else {
    // Aim for ~8 workgroups per CU over (page, KV head) work, in multiples of
    // 4 pages (one per wave), between 8 and 128 pages per partition.
    const int64_t cus = num_cus > 0 ? num_cus : 256;
    const int64_t target = cus * 8;
    int64_t p = (total * num_kv_heads + target - 1) / std::max<int64_t>(target, 1);
    p = (p + 3) / 4 * 4;
    ppp = int(std::min<int64_t>(std::max<int64_t>(p, 8), 128));
  }
  sched->batch = batch;
  sched->num_qo_heads = num_qo_heads;
  sched->num_kv_heads = num_kv_heads;
  sched->head_dim = head_dim;
  sched->page_size = page_size;
  sched->pages_per_partition = ppp;
  sched->max_partitions = std::max(1, (max_pages + ppp - 1) / ppp);
  sched->total_pages = int32_t(total);
  sched->num_empty = num_empty;
  sched->workspace_bytes =
      kvc_decode_workspace_bytes(batch, num_qo_heads, head_dim, sched->max_partitions);
  return ok();
}

extern "C" int kvc_batch_decode_run(
    const kvc_decode_schedule* sched, const void* q, int64_t q_batch_stride,
    const void* key_cache, const void* value_cache, int64_t cache_block_stride,
    int64_t cache_token_stride, int64_t num_blocks, const int32_t* indptr,
    const int32_t* indices, int64_t num_indices, const int32_t* last_page_len,
    float sm_scale, void* workspace, int64_t workspace_bytes, void* out,
    int64_t out_batch_stride, float* lse, void* stream) {
  KVC_REQUIRE(sched, KVC_ERR_INVALID_ARG, "null schedule");
  const int batch = sched->batch;
  if (batch == 0) return ok();
  KVC_REQUIRE(q && key_cache && value_cache && indptr && indices &&
                  last_page_len && out,
              KVC_ERR_INVALID_ARG, "null pointer");
  const int Hq = sched->num_qo_heads, Hkv = sched->num_kv_heads, D = sched->head_dim;
  KVC_REQUIRE(Hkv > 0 && Hq % Hkv == 0, KVC_ERR_INVALID_ARG, "bad head counts");
  const int group = Hq / Hkv;
  KVC_REQUIRE(sched->page_size == kPage, KVC_ERR_UNSUPPORTED, "page_size must be 16");
  KVC_REQUIRE(sched->pages_per_partition > 0 && sched->pages_per_partition % 4 == 0 &&
                  sched->max_partitions >= 1 && sched->max_partitions <= 65535,
              KVC_ERR_INVALID_ARG, "schedule not produced by kvc_decode_plan");
  KVC_REQUIRE(num_blocks > 0 && num_indices >= 0, KVC_ERR_INVALID_ARG,
              "bad num_blocks / num_indices");
  KVC_REQUIRE(cache_token_stride >= int64_t(Hkv) * D &&
                  cache_block_stride >= cache_token_stride * kPage,
              KVC_ERR_INVALID_ARG, "cache strides smaller than the block");
  KVC_REQUIRE(q_batch_stride >= int64_t(Hq) * D && out_batch_stride >= int64_t(Hq) * D,
              KVC_ERR_INVALID_ARG, "q/out batch stride smaller than Hq*head_dim");
  const int vec_bytes = D == 64 ? 8 : 16;
  KVC_REQUIRE(aligned(q, vec_bytes) && aligned(key_cache, vec_bytes) &&
                  aligned(value_cache, vec_bytes) &&
                  (q_batch_stride * 2) % vec_bytes == 0 &&
                  (cache_block_stride * 2) % vec_bytes == 0 &&
                  (cache_token_stride * 2) % vec_bytes == 0,
              KVC_ERR_ALIGNMENT, "q/cache pointers or strides not vector aligned");
  const int64_t need = kvc_decode_workspace_bytes(batch, Hq, D, sched->max_partitions);
  KVC_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), KVC_ERR_WORKSPACE,
              "decode workspace too small: need " + std::to_string(need) + " bytes");

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_stride = q_batch_stride;
  a.k_cache = static_cast<const uint16_t*>(key_cache);
  a.v_cache = static_cast<const uint16_t*>(value_cache);
  a.block_stride = cache_block_stride;
  a.token_stride = cache_token_stride;
  a.num_blocks = num_blocks;
  a.indptr = indptr;
  a.indices = indices;
  a.num_indices = num_indices;
  a.last_page_len = last_page_len;
  a.scale_log2 = sm_scale * kLog2e;
  a.num_kv_heads = Hkv;
  a.pages_per_part = sched->pages_per_partition;
  a.max_parts = sched->max_partitions;
  const int64_t rows = int64_t(batch) * Hq * sched->max_partitions;
  a.part_o = need ? static_cast<float*>(workspace) : nullptr;
  a.part_lse = need ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                              (rows * D * 4 + 255) / 256 * 256)
                    : nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.out_stride = out_batch_stride;
  a.lse = lse;
  hipStream_t s = static_cast<hipStream_t>(stream);

  bool launched = false;
  if (D == 128) launched = dispatch_group<128>(group, a, batch, s);
  else if (D == 64) launched = dispatch_group<64>(group, a, batch, s);
  else if (D == 256) launched = dispatch_group<256>(group, a, batch, s);
  KVC_REQUIRE(launched, KVC_ERR_UNSUPPORTED,
              "unsupported (group, head_dim) = (" + std::to_string(group) + ", " +
                  std::to_string(D) + ")");
  KVC_LAUNCH_CHECK();
  // Single-partition requests were written by the partition kernel; the merge
  // pass is needed for split requests and to zero empty ones.
  if (sched->max_partitions == 1 && sched->num_empty == 0) return ok();

  MergeArgs m;
  m.part_o = a.part_o;
  m.part_lse = a.part_lse;
  m.indptr = indptr;
  m.pages_per_part = a.pages_per_part;
  m.max_parts = a.max_parts;
  m.num_kv_heads = Hkv;
  m.group = group;
  m.out = a.out;
  m.out_stride = out_batch_stride;
  m.lse = lse;
  const dim3 mgrid{unsigned(Hq), unsigned(batch)};
  if (D == 128) decode_merge_kernel<128><<<mgrid, 64, 0, s>>>(m);
  else if (D == 64) decode_merge_kernel<64><<<mgrid, 64, 0, s>>>(m);
  else decode_merge_kernel<256><<<mgrid, 64, 0, s>>>(m);
  KVC_LAUNCH_CHECK();
  return ok();
}

extern "C" int kvc_merge_attention_states(const void* out1, const float* lse1,
                                          const void* out2, const float* lse2,
                                          int64_t n, int32_t head_dim, void* out,
                                          float* lse, void* stream) {
  KVC_REQUIRE(n >= 0 && head_dim > 0, KVC_ERR_INVALID_ARG, "bad shape");
  if (n == 0) return ok();
  KVC_REQUIRE(out1 && lse1 && out2 && lse2 && out, KVC_ERR_INVALID_ARG, "null pointer");
  KVC_REQUIRE(lse != lse1 && lse != lse2, KVC_ERR_INVALID_ARG,
              "lse must not alias lse1 or lse2");
  const int64_t total = n * head_dim;
  const int64_t grid = std::min<int64_t>((total + 255) / 256, 1 << 16);
  merge_states_kernel<<<dim3(unsigned(grid)), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(out1), lse1, static_cast<const uint16_t*>(out2), lse2,
      n, head_dim, static_cast<uint16_t*>(out), lse);
  KVC_LAUNCH_CHECK();
  return ok();
}
