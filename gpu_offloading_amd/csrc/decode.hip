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
// Decode is a GEMV: every K/V byte feeds only `group` query heads, so the
// kernels are HBM-bound and run on the VALU (no MFMA).
//
// Schedule (balanced split-KV, computed on the host by kvc_decode_plan like
// FlashInfer's plan()): the flattened page list indices[0 .. P) of the whole
// batch is cut into S segments of equal cost, S ~ the number of workgroups
// the GPU holds at once, so every workgroup streams about the same number of
// pages and all finish together whatever the spread of request lengths (a
// switch to another request inside a segment costs about one page more; see
// cut_segments).  A segment crosses request boundaries; the part of a request
// inside one segment is a "piece".  A request covered by one piece is written
// straight to the output; otherwise each piece leaves an fp32 partial +
// log2-sum-exp in the workspace and decode_merge_kernel folds them.
//
// head_dim 128 (the reference models) uses decode_lds_kernel<G, HPW>: grid
// (S, Hkv / HPW), one wave per KV head, HPW = 8 heads per workgroup when the
// heads divide evenly (else 1).  Every wave serves all `group` query heads of
// its KV head, so K/V are read from HBM exactly once.  The waves stage each
// page together: wave w loads 256 consecutive 16-byte chunks of the page's
// (token row x head slice) image (two whole 2 KB token rows for Mixtral), so
// the workgroup reads the page's K and V blocks as contiguous runs, into a
// double-buffered LDS tile; one barrier per page; the next two pages are in
// flight in two register stages meanwhile.  K/V are loaded with the
// non-temporal hint (read once; 5.7 -> 6.3 TB/s at 32K contexts).  Tile rows are padded by 16 B,
// which keeps both read patterns below free of LDS bank conflicts and makes
// every LDS address a lane base plus an immediate:
//   q.k : lane (token t, query head g) computes the whole 128-dim dot product
//         with v_dot2_f32_bf16 from 16 ds_read_b128 of row t (the four lanes
//         of a token read the same address); no cross-lane reduction;
//   p.v : lane l owns dims 2l, 2l+1 for every query head; per token one
//         ds_read_b32 of V and one broadcast read of p[t][0..G).
// Softmax statistics live per 16-lane DPP row (one query head per row).
// A wave's page ids are loaded once, one per lane (2 registers: up to 128
// pages per segment), and broadcast with v_readlane, so no dependent global
// load sits in the streaming loop.
//
// head_dim 64 and 256 use decode_reg_kernel: grid (S, ceil(Hkv / 4)), one
// wave per KV head, no barrier; K/V stay in registers: lane (row r, column c)
// holds 16 B of tokens r, r+4, r+8, r+12 and q.k is reduced over the 16 lanes
// of a DPP row.
#include "kvc_common.h"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

namespace kvc {
namespace {

constexpr int kThreads = 256;          // register kernel workgroup
constexpr int kWaves = kThreads / 64;  // KV heads per register-kernel workgroup
constexpr int kPage = 16;              // tokens per page (the engine's page_size)
constexpr int kTokPerRow = 4;          // register kernel: tokens of a page per 16-lane row
constexpr int kIdRegs = 2;             // page-id registers per lane
constexpr int kMaxSegPages = 64 * kIdRegs;
constexpr int kReadGroup = 4;  // LDS reads scheduled together
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
  const int32_t* indices;
  int64_t num_indices;
  const int4* segments;    // [S]: (first piece, end piece, first slot, pages)
  int32_t total_pages;     // pages of the whole batch
  int32_t num_segments;
  const int4* pieces;      // [N][2]: (request, first slot, end slot, partial or -1),
                           //         (request's last slot, its tokens, 0, 0)
  float scale_log2;        // sm_scale * log2(e)
  int32_t num_kv_heads;
  int32_t max_parts;
  float* part_o;           // [batch][Hkv][max_parts][G][D]
  float* part_lse;         // [batch][Hkv][max_parts][G]   (log2 domain)
  uint16_t* out;
  int64_t out_stride;      // elements between requests
  float* lse;              // [batch][Hq] natural log, may be null
  // Fused append (8 KV heads per workgroup): row b of new_k / new_v is
  // written as request b's last token before it is attended; null: none.
  const uint16_t* new_k;
  const uint16_t* new_v;
  int64_t new_k_stride;    // elements between requests
  int64_t new_v_stride;
};

// Pieces, counted from a segment's first, within which a fused append's
// request may end (the plan reports the most any segment needs).
constexpr int kNewMax = 4;

// Compiler-level ordering point for LDS traffic between lanes of one wave
// (the LDS unit itself executes one wave's instructions in order).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}


// First slot and page count of a segment, from its record (the plan's cuts
// balance pages and piece switches, so they do not follow from the index).
__device__ __forceinline__ void segment_span(const int4& segment, int& g0, int& n) {
  g0 = segment.z;
  n = min(segment.w, kMaxSegPages);
}

// Page ids of a segment: lane l of register r holds indices[g0 + l + 64 r].
// The registers are only ever indexed by constants (v_readlane picks the
// lane): a runtime index would turn them into a per-thread LDS array.
struct SegmentIds {
  int32_t r[kIdRegs];

  __device__ __forceinline__ void load(const DecodeArgs& a, int g0, int n, int lane) {
    // Clamped addresses, uniform branches: the loads issue back to back.
    const int64_t last = a.num_indices - 1;
#pragma unroll
    for (int i = 0; i < kIdRegs; ++i) {
      r[i] = -1;
      if (64 * i < n) {
        const int j = lane + 64 * i;
        const int64_t slot = int64_t(g0) + j;
        const int32_t v = a.indices[min(slot, last)];
        r[i] = (j < n && slot <= last) ? v : -1;
      }
    }
  }
  // Block id of the segment's j-th page (j uniform).
  __device__ __forceinline__ int32_t at(int j) const {
    const int l = j & 63;
    const int w = j >> 6;
    int32_t v = __builtin_amdgcn_readlane(r[0], l);
#pragma unroll
    for (int i = 1; i < kIdRegs; ++i) {
      const int32_t x = __builtin_amdgcn_readlane(r[i], l);
      v = w == i ? x : v;
    }
    return v;
  }
};

// The piece being streamed by a wave and what the page loop needs of it.
struct Piece {
  int4 desc;     // (request, first slot, end slot, partial index or -1)
  int req_last;  // slot of the request's final page
  int last_len;  // tokens in that page

  __device__ __forceinline__ void load(const DecodeArgs& a, int k) {
    desc = a.pieces[2 * k];
    const int4 tail = a.pieces[2 * k + 1];
    req_last = tail.x;
    last_len = min(max(tail.y, 0), kPage);
  }
  __device__ __forceinline__ int valid(int slot, int32_t blk, int64_t num_blocks) const {
    if (blk < 0 || blk >= num_blocks) return 0;
    return slot == req_last ? last_len : kPage;
  }
};

// Output of a finished piece for query head hq = h * group + g: the final
// bf16 row (a request covered by one piece) or an fp32 partial; `o` holds
// this lane's NDIM normalised values starting at dim d0.
template <int D, int NDIM>
__device__ __forceinline__ void write_piece(const DecodeArgs& a, const int4& pc, int h,
                                            int group, int g, int d0, const float (&o)[NDIM],
                                            float lse2, bool lse_lane) {
  const int b = pc.x;
  const int hq = h * group + g;
  if (pc.w < 0) {
    uint16_t* dst = a.out + int64_t(b) * a.out_stride + int64_t(hq) * D + d0;
    if constexpr (NDIM % 2 == 0) {
#pragma unroll
      for (int e = 0; e < NDIM; e += 2)
        *reinterpret_cast<uint32_t*>(dst + e) =
            uint32_t(f32_to_bf16(o[e])) | (uint32_t(f32_to_bf16(o[e + 1])) << 16);
    } else {
#pragma unroll
      for (int e = 0; e < NDIM; ++e) dst[e] = f32_to_bf16(o[e]);
    }
    if (a.lse && lse_lane)
      a.lse[int64_t(b) * a.num_kv_heads * group + hq] = lse2 * kLn2;
  } else {
    const int64_t pr = ((int64_t(b) * a.num_kv_heads + h) * a.max_parts + pc.w) * group + g;
    float* dst = a.part_o + pr * D + d0;
#pragma unroll
    for (int e = 0; e < NDIM; ++e) dst[e] = o[e];
    if (lse_lane) a.part_lse[pr] = lse2;
  }
}

// ---------------------------------------------------------------------------
// head_dim 128: LDS-staged kernel.
// ---------------------------------------------------------------------------
template <int G>
struct LdsCfg {
  static constexpr int QL = G > 4 ? G / 4 : 1;  // query heads per lane in q.k
  static constexpr int GP = G < 4 ? G : 4;      // distinct query heads over the 4 rows
  static constexpr int NS = G < 4 ? 4 / G : 1;  // lanes sharing one dot product
  static constexpr int CH = 16 / NS;            // 16-byte chunks of a K row per lane
};

// The LDS tile of one page for the HPW KV heads of a workgroup: K and V, 16
// token rows of HPW x 256 B, each row padded by 16 B.  With the pad, the 16
// rows read by one q.k instruction start on 16 different 4-bank groups, and
// every lane address is a lane base plus an immediate offset.
template <int HPW>
struct BlockTile {
  static constexpr int kRowBytes = HPW * 256 + 16;
  static constexpr int kRowChunks = kRowBytes / 16;
  uint4 k[kPage * kRowChunks];
  uint4 v[kPage * kRowChunks];
};

// Workgroup = HPW waves = HPW neighbouring KV heads of one segment.  The
// waves stage each page together: wave w loads 256 consecutive 16-byte chunks
// of the page's (token row x head slice) image, so the workgroup reads the
// block's rows as long contiguous runs (2 KB per token row for 8 heads), into
// a double-buffered tile; one barrier per page; then each wave computes its
// own head from the tile.
template <int G, int HPW>
__global__ __launch_bounds__(64 * HPW) void decode_lds_kernel(DecodeArgs a) {
  using C = LdsCfg<G>;
  using Tile = BlockTile<HPW>;
  constexpr int D = 128;
  constexpr int kSliceChunks = HPW * 16;  // 16-byte chunks per token row of the slice
  __shared__ Tile s_tile[2];
  __shared__ float s_p[HPW][kPage * 8];   // softmax weights p[token][query head]
  // Fused append: the new rows (K, V) of the requests that end inside the
  // segment, by piece index (8 heads per workgroup only).
  constexpr bool kAppend = HPW == 8;
  __shared__ uint4 s_new[kAppend ? kNewMax : 1][2][kAppend ? kSliceChunks : 1];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int h0 = blockIdx.y * HPW;  // first KV head of the workgroup
  const int h = h0 + wave;
  const int4 segment = a.segments[blockIdx.x];
  int g0, n;
  segment_span(segment, g0, n);
  int k = segment.x;
  const int k_end = segment.y;
  if (k >= k_end || n <= 0) return;  // uniform over the workgroup
  float* p_buf = s_p[wave];

  // q.k role: token t, query head gq (and gq + 4 when G == 8), dim split.
  const int t = lane & 15;
  const int row = lane >> 4;
  const int gq = row % C::GP;
  const int split = row / C::GP;
  // Staging role: chunk u of this lane is chunk q = 256 wave + 64 u + lane of
  // the page image (token q / kSliceChunks, 16-byte chunk q % kSliceChunks).
  uint32_t st_goff[4];
  int st_loff[4], st_tok[4];
  const uint32_t ts_bytes = uint32_t(a.token_stride * 2);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int q = 256 * wave + 64 * u + lane;
    st_tok[u] = q / kSliceChunks;
    const int cc = q % kSliceChunks;
    st_goff[u] = uint32_t(st_tok[u]) * ts_bytes + uint32_t(h0 * D * 2 + cc * 16);
    st_loff[u] = st_tok[u] * Tile::kRowChunks + cc;
  }
  const char* kbytes = reinterpret_cast<const char*>(a.k_cache);
  const char* vbytes = reinterpret_cast<const char*>(a.v_cache);
  const int64_t block_bytes = a.block_stride * 2;

  SegmentIds ids;
  ids.load(a, g0, n, lane);
  Piece pc;
  pc.load(a, k);
  const int k0 = k;
  const bool appending = kAppend && a.new_k != nullptr;
  // Thread i < 2 x kSliceChunks loads chunk i % kSliceChunks of the K (or V)
  // slice of each new row; the rows land in s_new after the first pages'
  // loads are issued.
  // The loads are issued on every path (a piece past the segment's last
  // re-reads that one's row), so the compiler's count of loads in flight stays
  // exact and staging s_new does not wait for the first pages' loads.
  uint4 nrow[kAppend ? kNewMax : 1];
#pragma unroll
  for (int i = 0; i < (kAppend ? kNewMax : 1); ++i) nrow[i] = make_uint4(0, 0, 0, 0);
  if constexpr (kAppend) {
    if (appending) {
      const int is_v = (threadIdx.x & (2 * kSliceChunks - 1)) >= kSliceChunks;
      const int cc = threadIdx.x & (kSliceChunks - 1);
#pragma unroll
      for (int i = 0; i < kNewMax; ++i) {
        const int b = a.pieces[2 * min(k + i, k_end - 1)].x;
        const uint16_t* src = is_v ? a.new_v + int64_t(b) * a.new_v_stride
                                   : a.new_k + int64_t(b) * a.new_k_stride;
        nrow[i] = reinterpret_cast<const uint4*>(src + h0 * D)[cc];
      }
    }
  }

  uint32_t qw[C::QL][C::CH * 4];
  auto load_q = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) {
      const uint4* qp = reinterpret_cast<const uint4*>(
          a.q + int64_t(b) * a.q_stride + int64_t(h * G + gq + 4 * ql) * D + split * C::CH * 8);
#pragma unroll
      for (int i = 0; i < C::CH; ++i) {
        const uint4 x = qp[i];
        qw[ql][4 * i + 0] = x.x;
        qw[ql][4 * i + 1] = x.y;
        qw[ql][4 * i + 2] = x.z;
        qw[ql][4 * i + 3] = x.w;
      }
    }
  };
  float m_run[C::QL], l_run[C::QL], acc[G][2];
  auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) {
      m_run[ql] = kNegBig;
      l_run[ql] = 0.f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;
  };
  auto finalize = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float l = readlane_f(l_run[g / 4], 16 * (g % 4));
      const float m = readlane_f(m_run[g / 4], 16 * (g % 4));
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const float o[2] = {acc[g][0] * inv, acc[g][1] * inv};
      write_piece<D, 2>(a, pc.desc, h, G, g, 2 * lane, o,
                        l > 0.f ? m + fast_log2(l) : -INFINITY, lane == 0);
    }
  };

  // Two register stages: while page j is consumed, pages j+1 and j+2 are in
  // flight (2 x 8 KB per wave, 2 x 8 KB x HPW per workgroup).
  struct Stage {
    uint4 k[4], v[4];
  };
  auto issue = [&](Stage& r, int32_t blk) __attribute__((always_inline)) {
    // Uniform block base (SGPRs) + 32-bit lane offset.
    const char* kb = kbytes + int64_t(blk) * block_bytes;
    const char* vb = vbytes + int64_t(blk) * block_bytes;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      r.k[u] = load_stream(kb + st_goff[u]);
      r.v[u] = load_stream(vb + st_goff[u]);
    }
  };
  auto safe_id = [&](int32_t id) __attribute__((always_inline)) { return (id >= 0 && id < a.num_blocks) ? id : 0; };
  auto stage_tile = [&](Stage& r, Tile& tile, int valid) __attribute__((always_inline)) {
    if (valid < kPage) {
      // Rows past the end may hold anything (even NaN bits): stage zeros so
      // that 0 * v stays 0.
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (st_tok[u] >= valid) r.k[u] = r.v[u] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      tile.k[st_loff[u]] = r.k[u];
      tile.v[st_loff[u]] = r.v[u];
    }
  };
  auto consume = [&](const Tile& tile, int valid) __attribute__((always_inline)) {
    // q.k: lane (t, gq) over its chunks of K row t, head `wave` of the tile.
    float dots[C::QL];
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) dots[ql] = 0.f;
    const uint4* krow = tile.k + t * Tile::kRowChunks + wave * 16 + split * C::CH;
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const uint4 kv = krow[i];
#pragma unroll
      for (int ql = 0; ql < C::QL; ++ql) {
        dots[ql] = dot2_bf16(qw[ql][4 * i + 0], kv.x, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * i + 1], kv.y, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * i + 2], kv.z, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * i + 3], kv.w, dots[ql]);
      }
      // Keep a bounded number of LDS reads in flight: hoisting all of them
      // would cost registers, and with them a wave per SIMD.
      if ((i + 1) % kReadGroup == 0) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int off = 16 * C::GP; off < 64; off <<= 1)
#pragma unroll
      for (int ql = 0; ql < C::QL; ++ql) dots[ql] += __shfl_xor(dots[ql], off);

    // Online softmax per row (one query head per 16-lane row).
    const bool live = t < valid;
    float alpha[C::QL];
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) {
      const float s = live ? dots[ql] * a.scale_log2 : kNegBig;
      const float m_new = fmaxf(m_run[ql], row16_max(s));
      const float p = live ? fast_exp2(s - m_new) : 0.f;
      alpha[ql] = fast_exp2(m_run[ql] - m_new);
      l_run[ql] = fmaf(l_run[ql], alpha[ql], row16_sum(p));
      m_run[ql] = m_new;
      if (row < C::GP) p_buf[t * G + gq + 4 * ql] = p;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float al = readlane_f(alpha[g / 4], 16 * (g % 4));
      acc[g][0] *= al;
      acc[g][1] *= al;
    }
    wave_lds_fence();

    // p.v over the 16 tokens of the page (rows past `valid` are zero).
    const uint32_t* vcol = reinterpret_cast<const uint32_t*>(tile.v + wave * 16) + lane;
#pragma unroll
    for (int tt = 0; tt < kPage; ++tt) {
      const uint32_t vw = vcol[tt * Tile::kRowChunks * 4];
      const float v0 = bf16lo(vw);
      const float v1 = bf16hi(vw);
      float pg[G];
      if constexpr (G >= 4) {
#pragma unroll
        for (int q4 = 0; q4 < G / 4; ++q4) {
          const float4 x = reinterpret_cast<const float4*>(p_buf + tt * G)[q4];
          pg[4 * q4 + 0] = x.x;
          pg[4 * q4 + 1] = x.y;
          pg[4 * q4 + 2] = x.z;
          pg[4 * q4 + 3] = x.w;
        }
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) pg[g] = p_buf[tt * G + g];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        acc[g][0] = fmaf(pg[g], v0, acc[g][0]);
        acc[g][1] = fmaf(pg[g], v1, acc[g][1]);
      }
      if ((tt + 1) % kReadGroup == 0) __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Page j: stage it into tile j%2, refill its register stage with page j+2,
  // wait for the whole workgroup's part of the tile (one barrier per page:
  // every wave has also finished reading the tile's previous page j-2),
  // consume, and close the piece if page j is its last.
  auto step = [&](int j, Stage& r, int32_t& id, Tile& tile) __attribute__((always_inline)) {
    const int slot = g0 + j;
    const int valid = pc.valid(slot, id, a.num_blocks);
    if constexpr (kAppend) {
      // The request's last page: its new token row comes from s_new (the
      // loaded row is stale) and is written to the cache.
      if (appending && slot == pc.req_last && valid > 0 && k - k0 < kNewMax) {
        const int tnew = valid - 1;
        const int i = k - k0;
        char* kdst = const_cast<char*>(kbytes) + int64_t(id) * block_bytes;
        char* vdst = const_cast<char*>(vbytes) + int64_t(id) * block_bytes;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (st_tok[u] == tnew) {
            const int cc = st_loff[u] - st_tok[u] * Tile::kRowChunks;
            r.k[u] = s_new[i][0][cc];
            r.v[u] = s_new[i][1][cc];
            store_stream(kdst + st_goff[u], r.k[u]);
            store_stream(vdst + st_goff[u], r.v[u]);
          }
        }
      }
    }
    stage_tile(r, tile, valid);
    if (j + 2 < n) {
      id = ids.at(j + 2);
      issue(r, safe_id(id));
    }
    __syncthreads();
    consume(tile, valid);
    wave_lds_fence();
    if (slot + 1 == pc.desc.z) {
      finalize();
      if (++k < k_end) {
        pc.load(a, k);
        load_q(pc.desc.x);
        reset();
      }
    }
  };

  load_q(pc.desc.x);
  reset();
  Stage ra, rb;
  int32_t ida = ids.at(0), idb = 0;
  issue(ra, safe_id(ida));
  if (n > 1) {
    idb = ids.at(1);
    issue(rb, safe_id(idb));
  }
  if constexpr (kAppend) {
    if (appending) {
      if (threadIdx.x < 2 * kSliceChunks) {
        const int is_v = threadIdx.x >= kSliceChunks;
        const int cc = threadIdx.x & (kSliceChunks - 1);
#pragma unroll
        for (int i = 0; i < kNewMax; ++i) s_new[i][is_v][cc] = nrow[i];
      }
      __syncthreads();
    }
  }
  for (int j = 0; j < n; j += 2) {
    step(j, ra, ida, s_tile[0]);
    if (j + 1 < n) step(j + 1, rb, idb, s_tile[1]);
  }
}

// ---------------------------------------------------------------------------
// head_dim 128, small batches: one workgroup per (request, KV head), its
// kSmallWaves waves splitting the request's pages (wave w takes pages w,
// w + kSmallWaves, ...), the waves' softmax states merged in LDS.  One launch,
// no partials in memory and no merge kernel: for batches whose requests fit
// in kSmallMaxPages pages but would otherwise be cut into one-page segments
// and merged (batch 1 at a 128-token context: 9 pages).  The plan image holds
// one segment and one piece per request (empty requests included), so the
// request's record sits at piece index b.
// ---------------------------------------------------------------------------
constexpr int kSmallWaves = 8;
constexpr int kSmallMaxPages = 2 * kSmallWaves;

template <int G>
__global__ __launch_bounds__(64 * kSmallWaves) void decode_small_kernel(DecodeArgs a) {
  using C = LdsCfg<G>;
  using Tile = BlockTile<1>;
  constexpr int D = 128;
  constexpr int kPagesPerWave = kSmallMaxPages / kSmallWaves;
  __shared__ Tile s_tile[kSmallWaves];
  __shared__ float s_p[kSmallWaves][kPage * 8];
  __shared__ float s_m[kSmallWaves][G];
  __shared__ float s_l[kSmallWaves][G];
  __shared__ float s_o[kSmallWaves][G][D];

  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int4 desc = a.pieces[2 * b];        // (request, first slot, end slot, -1)
  const int4 tail = a.pieces[2 * b + 1];    // (request's last slot, its tokens, 0, 0)
  const int first = desc.y;
  const int npages = min(desc.z - desc.y, kSmallMaxPages);
  const int last_len = min(max(tail.y, 0), kPage);
  Tile& tile = s_tile[wave];
  float* p_buf = s_p[wave];

  const int t = lane & 15;
  const int row = lane >> 4;
  const int gq = row % C::GP;
  const int split = row / C::GP;
  // Staging: chunk u of this lane is chunk 64 u + lane of the (16 tokens x
  // 256 B) image of head h in a page: token (64 u + lane) / 16, chunk lane % 16.
  const int cc = lane & 15;
  const uint32_t ts_bytes = uint32_t(a.token_stride * 2);
  uint32_t st_goff[4];
  int st_tok[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    st_tok[u] = (64 * u + lane) >> 4;
    st_goff[u] = uint32_t(st_tok[u]) * ts_bytes + uint32_t(h * D * 2 + cc * 16);
  }
  const char* kbytes = reinterpret_cast<const char*>(a.k_cache);
  const char* vbytes = reinterpret_cast<const char*>(a.v_cache);
  const int64_t block_bytes = a.block_stride * 2;

  // This wave's pages, their ids and their loads, all issued up front.
  struct Stage {
    uint4 k[4], v[4];
  };
  Stage st[kPagesPerWave];
  int32_t ids[kPagesPerWave];
#pragma unroll
  for (int i = 0; i < kPagesPerWave; ++i) {
    const int j = wave + kSmallWaves * i;
    ids[i] = -1;
    if (j < npages) {
      const int64_t slot = int64_t(first) + j;
      ids[i] = slot < a.num_indices ? a.indices[slot] : -1;
    }
  }
#pragma unroll
  for (int i = 0; i < kPagesPerWave; ++i) {
    const int32_t id = (ids[i] >= 0 && ids[i] < a.num_blocks) ? ids[i] : 0;
    const char* kb = kbytes + int64_t(id) * block_bytes;
    const char* vb = vbytes + int64_t(id) * block_bytes;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      st[i].k[u] = make_uint4(0, 0, 0, 0);
      st[i].v[u] = make_uint4(0, 0, 0, 0);
    }
    if (wave + kSmallWaves * i < npages) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        st[i].k[u] = load_stream(kb + st_goff[u]);
        st[i].v[u] = load_stream(vb + st_goff[u]);
      }
    }
  }
  // Fused append: lane chunk cc of head h of the request's new K / V row.
  const bool appending = a.new_k != nullptr && npages > 0 && last_len > 0;
  uint4 nk = make_uint4(0, 0, 0, 0), nv = make_uint4(0, 0, 0, 0);
  if (appending) {
    nk = reinterpret_cast<const uint4*>(a.new_k + int64_t(b) * a.new_k_stride + h * D)[cc];
    nv = reinterpret_cast<const uint4*>(a.new_v + int64_t(b) * a.new_v_stride + h * D)[cc];
  }

  uint32_t qw[C::QL][C::CH * 4];
#pragma unroll
  for (int ql = 0; ql < C::QL; ++ql) {
    const uint4* qp = reinterpret_cast<const uint4*>(
        a.q + int64_t(b) * a.q_stride + int64_t(h * G + gq + 4 * ql) * D + split * C::CH * 8);
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const uint4 x = qp[i];
      qw[ql][4 * i + 0] = x.x;
      qw[ql][4 * i + 1] = x.y;
      qw[ql][4 * i + 2] = x.z;
      qw[ql][4 * i + 3] = x.w;
    }
  }
  float m_run[C::QL], l_run[C::QL], acc[G][2];
#pragma unroll
  for (int ql = 0; ql < C::QL; ++ql) {
    m_run[ql] = kNegBig;
    l_run[ql] = 0.f;
  }
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;

#pragma unroll
  for (int i = 0; i < kPagesPerWave; ++i) {
    const int j = wave + kSmallWaves * i;
    if (j >= npages) break;  // uniform over the wave
    const int slot = first + j;
    const int32_t id = ids[i];
    const bool ok = id >= 0 && id < a.num_blocks;
    const int valid = !ok ? 0 : (slot == tail.x ? last_len : kPage);
    Stage& r = st[i];
    if (appending && slot == tail.x && ok) {
      // The request's last page: its new token row (row valid - 1) comes
      // from the step's rows and is written to the cache.
      char* kdst = const_cast<char*>(kbytes) + int64_t(id) * block_bytes;
      char* vdst = const_cast<char*>(vbytes) + int64_t(id) * block_bytes;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (st_tok[u] == valid - 1) {
          r.k[u] = nk;
          r.v[u] = nv;
          store_stream(kdst + st_goff[u], nk);
          store_stream(vdst + st_goff[u], nv);
        }
      }
    }
    // Stage the page into this wave's tile (rows past `valid` as zeros).
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool live = st_tok[u] < valid;
      tile.k[st_tok[u] * Tile::kRowChunks + cc] = live ? r.k[u] : make_uint4(0, 0, 0, 0);
      tile.v[st_tok[u] * Tile::kRowChunks + cc] = live ? r.v[u] : make_uint4(0, 0, 0, 0);
    }
    wave_lds_fence();
    // q.k: lane (t, gq) over its chunks of K row t.
    float dots[C::QL];
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) dots[ql] = 0.f;
    const uint4* krow = tile.k + t * Tile::kRowChunks + split * C::CH;
#pragma unroll
    for (int c = 0; c < C::CH; ++c) {
      const uint4 kv = krow[c];
#pragma unroll
      for (int ql = 0; ql < C::QL; ++ql) {
        dots[ql] = dot2_bf16(qw[ql][4 * c + 0], kv.x, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * c + 1], kv.y, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * c + 2], kv.z, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * c + 3], kv.w, dots[ql]);
      }
    }
#pragma unroll
    for (int off = 16 * C::GP; off < 64; off <<= 1)
#pragma unroll
      for (int ql = 0; ql < C::QL; ++ql) dots[ql] += __shfl_xor(dots[ql], off);
    const bool live = t < valid;
    float alpha[C::QL];
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) {
      const float s = live ? dots[ql] * a.scale_log2 : kNegBig;
      const float m_new = fmaxf(m_run[ql], row16_max(s));
      const float p = live ? fast_exp2(s - m_new) : 0.f;
      alpha[ql] = fast_exp2(m_run[ql] - m_new);
      l_run[ql] = fmaf(l_run[ql], alpha[ql], row16_sum(p));
      m_run[ql] = m_new;
      if (row < C::GP) p_buf[t * G + gq + 4 * ql] = p;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float al = readlane_f(alpha[g / 4], 16 * (g % 4));
      acc[g][0] *= al;
      acc[g][1] *= al;
    }
    wave_lds_fence();
    // p.v over the page's rows: all 16 for a full page, else four at a time
    // up to `valid` (rows past it have p = 0 and zero V rows, so leaving
    // them out changes nothing).
    const uint32_t* vcol = reinterpret_cast<const uint32_t*>(tile.v) + lane;
    auto pv_row = [&](int tt) {
      const uint32_t vw = vcol[tt * Tile::kRowChunks * 4];
      const float v0 = bf16lo(vw);
      const float v1 = bf16hi(vw);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pg = p_buf[tt * G + g];
        acc[g][0] = fmaf(pg, v0, acc[g][0]);
        acc[g][1] = fmaf(pg, v1, acc[g][1]);
      }
    };
    if (valid == kPage) {
#pragma unroll
      for (int tt = 0; tt < kPage; ++tt) pv_row(tt);
    } else {
      for (int t4 = 0; t4 < valid; t4 += 4) {
#pragma unroll
        for (int tt = t4; tt < t4 + 4; ++tt) pv_row(tt);
      }
    }
    wave_lds_fence();  // the tile and p_buf are rewritten by the next page
  }

  // The waves' states (log2 domain) into LDS, then one merged output row per
  // query head; lanes cover (query head, dim).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float l = readlane_f(l_run[g / 4], 16 * (g % 4));
    const float m = readlane_f(m_run[g / 4], 16 * (g % 4));
    if (lane == 0) {
      s_m[wave][g] = m;
      s_l[wave][g] = l;
    }
    s_o[wave][g][2 * lane] = acc[g][0];
    s_o[wave][g][2 * lane + 1] = acc[g][1];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * D; e += 64 * kSmallWaves) {
    const int g = e / D;
    const int d = e - g * D;
    float mx = kNegBig;
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w)
      if (s_l[w][g] > 0.f) mx = fmaxf(mx, s_m[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w) {
      if (s_l[w][g] > 0.f) {
        const float wt = fast_exp2(s_m[w][g] - mx);
        L = fmaf(s_l[w][g], wt, L);
        O = fmaf(s_o[w][g][d], wt, O);
      }
    }
    const int hq = h * G + g;
    a.out[int64_t(b) * a.out_stride + int64_t(hq) * D + d] = f32_to_bf16(L > 0.f ? O / L : 0.f);
    if (a.lse && d == 0)
      a.lse[int64_t(b) * a.num_kv_heads * G + hq] =
          L > 0.f ? (mx + fast_log2(L)) * kLn2 : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// head_dim 64 / 256: register kernel.
// ---------------------------------------------------------------------------
// Load the D/16 bf16 elements one lane owns (D/32 32-bit words).
template <int D, bool kStream = false>
__device__ __forceinline__ void load_slice(uint32_t (&w)[D / 32], const uint16_t* p) {
  if constexpr (D == 64) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    w[0] = x.x; w[1] = x.y;
  } else {
    static_assert(D == 128 || D == 256, "head_dim must be 64, 128 or 256");
#pragma unroll
    for (int i = 0; i < D / 128; ++i) {
      const uint4 x = kStream ? load_stream(reinterpret_cast<const uint4*>(p) + i)
                              : reinterpret_cast<const uint4*>(p)[i];
      w[4 * i + 0] = x.x; w[4 * i + 1] = x.y; w[4 * i + 2] = x.z; w[4 * i + 3] = x.w;
    }
  }
}

template <int D>
struct PageRegs {
  uint32_t k[kTokPerRow][D / 32];
  uint32_t v[kTokPerRow][D / 32];
};

template <int D>
__device__ __forceinline__ void load_page_regs(const DecodeArgs& a, PageRegs<D>& r,
                                               int32_t blk, int64_t lane_off) {
  const int64_t base = int64_t(blk) * a.block_stride + lane_off;
#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j)
    load_slice<D, true>(r.k[j], a.k_cache + base + int64_t(j) * kTokPerRow * a.token_stride);
#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j)
    load_slice<D, true>(r.v[j], a.v_cache + base + int64_t(j) * kTokPerRow * a.token_stride);
}

// Fold one page into the row's online-softmax state.
template <int G, int D>
__device__ __forceinline__ void consume_page_regs(const uint32_t (&qw)[G][D / 32],
                                                  PageRegs<D>& r, int valid, int row,
                                                  float scale_log2, float (&m)[G],
                                                  float (&l)[G], float (&acc)[G][D / 16]) {
  constexpr int W = D / 32;
  if (valid < kPage) {
#pragma unroll
    for (int j = 0; j < kTokPerRow; ++j)
      if (row + kTokPerRow * j >= valid)
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
      d = row16_sum(d) * scale_log2;
      s[j][g] = row + kTokPerRow * j < valid ? d : kNegBig;
    }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = s[0][g];
#pragma unroll
    for (int j = 1; j < kTokPerRow; ++j) mx = fmaxf(mx, s[j][g]);
    const float m_new = fmaxf(m[g], mx);
    const float alpha = fast_exp2(m[g] - m_new);
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < kTokPerRow; ++j) {
      s[j][g] = row + kTokPerRow * j < valid ? fast_exp2(s[j][g] - m_new) : 0.f;
      psum += s[j][g];
    }
    l[g] = fmaf(l[g], alpha, psum);
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
        acc[g][2 * w] = fmaf(s[j][g], v0, acc[g][2 * w]);
        acc[g][2 * w + 1] = fmaf(s[j][g], v1, acc[g][2 * w + 1]);
      }
    }
}

template <int G, int D>
__global__ __launch_bounds__(kThreads) void decode_reg_kernel(DecodeArgs a) {
  constexpr int W = D / 32;
  constexpr int E = D / 16;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * kWaves + wave;
  if (h >= a.num_kv_heads) return;
  const int4 segment = a.segments[blockIdx.x];
  int g0, n;
  segment_span(segment, g0, n);
  int k = segment.x;
  const int k_end = segment.y;
  if (k >= k_end || n <= 0) return;
  const int row = lane >> 4;
  const int col = lane & 15;
  const int64_t lane_off = int64_t(row) * a.token_stride + int64_t(h) * D + col * E;

  SegmentIds ids;
  ids.load(a, g0, n, lane);
  Piece pc;
  pc.load(a, k);

  uint32_t qw[G][W];
  auto load_q = [&](int b) __attribute__((always_inline)) {
    const uint16_t* qb = a.q + int64_t(b) * a.q_stride + int64_t(h) * G * D + col * E;
#pragma unroll
    for (int g = 0; g < G; ++g) load_slice<D>(qw[g], qb + g * D);
  };
  float m[G], l[G], acc[G][E];
  auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = kNegBig;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
    }
  };
  auto finalize = [&]() __attribute__((always_inline)) {
    // Merge the four rows (lanes c, c+16, c+32, c+48 hold the same dims).
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
    if (row == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;
        float o[E];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = acc[g][e] * inv;
        write_piece<D, E>(a, pc.desc, h, G, g, col * E, o,
                          l[g] > 0.f ? m[g] + fast_log2(l[g]) : -INFINITY, col == 0);
      }
    }
  };

  // Two register sets: page j is consumed while page j+1 is in flight.
  auto safe = [&](int32_t id) __attribute__((always_inline)) { return (id >= 0 && id < a.num_blocks) ? id : 0; };
  PageRegs<D> ra, rb;
  auto step = [&](int j, PageRegs<D>& cur, int32_t id, PageRegs<D>& nxt, int32_t& nid) __attribute__((always_inline)) {
    const int slot = g0 + j;
    if (j + 1 < n) {
      nid = ids.at(j + 1);
      load_page_regs<D>(a, nxt, safe(nid), lane_off);
    }
    consume_page_regs<G, D>(qw, cur, pc.valid(slot, id, a.num_blocks), row, a.scale_log2,
                            m, l, acc);
    if (slot + 1 == pc.desc.z) {
      finalize();
      if (++k < k_end) {
        pc.load(a, k);
        load_q(pc.desc.x);
        reset();
      }
    }
  };

  load_q(pc.desc.x);
  reset();
  int32_t ida = ids.at(0), idb = 0;
  load_page_regs<D>(a, ra, safe(ida), lane_off);
  for (int j = 0; j < n; j += 2) {
    step(j, ra, ida, rb, idb);
    if (j + 1 < n) step(j + 1, rb, idb, ra, ida);
  }
}

// ---------------------------------------------------------------------------
// Split-K merge.
// ---------------------------------------------------------------------------
struct MergeArgs {
  const float* part_o;
  const float* part_lse;
  const int32_t* req_nparts;
  int32_t max_parts;
  int32_t num_kv_heads;
  int32_t group;
  uint16_t* out;
  int64_t out_stride;
  float* lse;
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// One wave per (request, query head).  The partials of the first kSpecParts
// pieces and the log2-sum-exps are loaded together with the request's piece
// count (all inside the max_parts rows the workspace holds for the request),
// so the common case costs one memory round trip; lane p weighs piece p and
// every lane folds its D/64 dims.  Requests with a single piece were finished
// by the streaming kernel; requests with no pages get a zero output and
// lse = -inf.
//
// With no split request in the batch (max_parts == 1) the launch only zeroes
// the empty requests and the workspace is absent (part_o == part_lse ==
// null): then no partial is read, and every request counts at most one
// piece.
constexpr int kSpecParts = 16;

template <int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(MergeArgs a) {
  constexpr int EPL = D / 64;  // dims per lane
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int G = a.group;
  const int Hq = a.num_kv_heads * G;
  const int h = hq / G;
  const int g = hq - h * G;
  const bool have_parts = a.part_o != nullptr && a.part_lse != nullptr;  // uniform
  const int max_parts = have_parts ? a.max_parts : 1;
  const int64_t base = (int64_t(b) * a.num_kv_heads + h) * max_parts;
  const int64_t lse0 = base * G + g;  // piece p at part_lse[lse0 + p * G]
  const int nparts_raw = a.req_nparts[b];
  const int nspec = have_parts ? min(max_parts, kSpecParts) : 0;
  const float lse_spec = (have_parts && lane < min(max_parts, 64))
                             ? a.part_lse[lse0 + int64_t(lane) * G] : -INFINITY;
  float po[kSpecParts][EPL];
#pragma unroll
  for (int p = 0; p < kSpecParts; ++p) {
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      po[p][e] = p < nspec ? a.part_o[((base + p) * G + g) * D + lane * EPL + e] : 0.f;
  }
  const int nparts = min(nparts_raw, max_parts);
  if (nparts == 1) return;
  const float* lp = have_parts ? a.part_lse + lse0 : nullptr;  // read only when nparts > 64
  uint16_t* out = a.out + int64_t(b) * a.out_stride + int64_t(hq) * D;

  float mx = lane < nparts ? lse_spec : -INFINITY;
  for (int p = 64 + lane; p < nparts; p += 64) mx = fmaxf(mx, lp[int64_t(p) * G]);
  mx = wave_max(mx);
  if (nparts <= 0 || mx == -INFINITY) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) out[lane * EPL + e] = 0;
    if (a.lse && lane == 0) a.lse[int64_t(b) * Hq + hq] = -INFINITY;
    return;
  }
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  const float w0 = lane < nparts ? fast_exp2(lse_spec - mx) : 0.f;
  float S = w0;
  if (nparts <= kSpecParts) {
#pragma unroll
    for (int p = 0; p < kSpecParts; ++p) {
      if (p < nparts) {
        const float wp = readlane_f(w0, p);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = fmaf(wp, po[p][e], acc[e]);
      }
    }
  } else {
    for (int q0 = 0; q0 < nparts; q0 += 64) {
      const float w = q0 == 0 ? w0
                              : (q0 + lane < nparts
                                     ? fast_exp2(lp[int64_t(q0 + lane) * G] - mx) : 0.f);
      if (q0 > 0) S += w;
      const int cnt = min(64, nparts - q0);
      for (int j = 0; j < cnt; ++j) {
        const float wj = readlane_f(w, j);
        const float* src = a.part_o + ((base + q0 + j) * G + g) * D + lane * EPL;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = fmaf(wj, src[e], acc[e]);
      }
    }
  }
  S = wave_sum(S);
  const float inv = 1.f / S;
#pragma unroll
  for (int e = 0; e < EPL; ++e) out[lane * EPL + e] = f32_to_bf16(acc[e] * inv);
  if (a.lse && lane == 0) a.lse[int64_t(b) * Hq + hq] = (mx + fast_log2(S)) * kLn2;
}

// Segment cuts of the flattened page list [0, total): cut[s] is segment s's
// first page, cut[segs] = total.  The segments cost the same, a page counting
// kPageCost and every request that starts strictly inside a segment
// kSwitchCost more: at such a piece switch the workgroup loads the next
// request's record and q while its page pipeline drains by about one page
// (a 35-page segment with one switch was measured 2.5 us = 1.15 pages slower
// than one without).  Every segment keeps at least one page; if the balanced
// cuts would give a segment more than kMaxSegPages pages, equal page counts
// are used instead.
constexpr int64_t kPageCost = 8;
constexpr int64_t kSwitchCost = 9;

std::vector<int64_t> cut_segments(const int32_t* indptr, int batch, int64_t total,
                                  int64_t segs) {
  std::vector<int64_t> cut(size_t(segs) + 1);
  cut[0] = 0;
  cut[size_t(segs)] = total;
  if (segs <= 1) return cut;
  // first pages of the requests after the first non-empty one
  std::vector<int64_t> starts;
  for (int b = 1; b < batch; ++b)
    if (indptr[b + 1] > indptr[b] && indptr[b] > 0) starts.push_back(indptr[b]);
  // F(x) = cost of pages [0, x): cut s goes where F is nearest to s/segs of
  // the total, so a cut can land exactly on a request's first page (which
  // then costs no switch: F counts it in the segment it starts).
  const __int128 T = __int128(kPageCost) * total + __int128(kSwitchCost) * int64_t(starts.size());
  auto F = [&](int64_t x, int64_t below) { return __int128(kPageCost) * x + __int128(kSwitchCost) * below; };
  int64_t x = 0, below = 0;  // below = starts < x
  size_t next = 0;
  bool ok = true;
  for (int64_t s = 1; s < segs; ++s) {
    const __int128 target = __int128(s) * T / segs;
    while (x < total && F(x, below) < target) {
      ++x;
      while (next < starts.size() && starts[next] < x) ++below, ++next;
    }
    // x is the first page with F(x) >= target; x - 1 may be nearer
    int64_t pick = x;
    if (x > 0) {
      const int64_t below_prev = below - ((next > 0 && starts[next - 1] == x - 1) ? 1 : 0);
      if (target - F(x - 1, below_prev) < F(x, below) - target) pick = x - 1;
    }
    cut[size_t(s)] = std::min(std::max(pick, cut[size_t(s) - 1] + 1), total - (segs - s));
    ok = ok && cut[size_t(s)] - cut[size_t(s) - 1] <= kMaxSegPages;
  }
  ok = ok && total - cut[size_t(segs) - 1] <= kMaxSegPages;
  if (!ok)
    for (int64_t s = 1; s < segs; ++s) cut[size_t(s)] = s * total / segs;
  return cut;
}

// KV heads per workgroup of the streaming kernel: 8 (one block-row slice of
// 2 KB per token) for the head_dim-128 kernel when the heads divide evenly
// and the register budget allows two waves per SIMD, else one; the register
// kernel always groups 4 heads (and idles waves past the last head).
int heads_per_workgroup(int group, int head_dim, int num_kv_heads) {
  if (head_dim != 128) return 4;
  return (group <= 4 && num_kv_heads % 8 == 0) ? 8 : 1;
}

// Workgroups of the streaming kernel one CU holds at once (LDS- or
// register-limited; from the compiled kernels' resources), used to size the
// schedule.
int resident_workgroups_per_cu(int group, int head_dim, int hpw) {
  if (head_dim == 128) return hpw == 8 ? 1 : (group == 8 ? 4 : 8);
  return group <= 2 ? 2 : 1;
}

template <int G, int D>
void launch_segments(const DecodeArgs& a, int segments, int head_groups, int hpw,
                     hipStream_t s) {
  const dim3 grid{unsigned(segments), unsigned(head_groups)};
  if constexpr (D == 128) {
    if constexpr (G <= 4) {
      if (hpw == 8) {
        decode_lds_kernel<G, 8><<<grid, 64 * 8, 0, s>>>(a);
        return;
      }
    }
    decode_lds_kernel<G, 1><<<grid, 64, 0, s>>>(a);
  } else {
    decode_reg_kernel<G, D><<<grid, kThreads, 0, s>>>(a);
  }
}

template <int D>
bool dispatch_group(int group, const DecodeArgs& a, int segments, int head_groups, int hpw,
                    hipStream_t s) {
  switch (group) {
    case 1: launch_segments<1, D>(a, segments, head_groups, hpw, s); return true;
    case 2: launch_segments<2, D>(a, segments, head_groups, hpw, s); return true;
    case 4: launch_segments<4, D>(a, segments, head_groups, hpw, s); return true;
    case 8: launch_segments<8, D>(a, segments, head_groups, hpw, s); return true;
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

extern "C" int64_t kvc_decode_plan_ints(int32_t batch, int32_t num_segments) {
  if (batch < 0 || num_segments < 0) return -1;
  return 4 * int64_t(num_segments) + 8 * (int64_t(num_segments) + batch) + batch;
}

extern "C" int kvc_decode_plan(const int32_t* indptr_host, const int32_t* last_page_len_host,
                               int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                               int32_t head_dim, int32_t page_size,
                               int32_t num_segments_hint, int32_t num_cus,
                               kvc_decode_schedule* sched, int32_t* plan_host,
                               int64_t plan_capacity) {
  KVC_REQUIRE(sched, KVC_ERR_INVALID_ARG, "null schedule");
  KVC_REQUIRE(batch >= 0 && batch <= 65535, KVC_ERR_INVALID_ARG,
              "batch must be in [0, 65535]");
  KVC_REQUIRE(batch == 0 || (indptr_host && last_page_len_host), KVC_ERR_INVALID_ARG,
              "null indptr or last_page_len");
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
  KVC_REQUIRE(batch == 0 || indptr_host[0] == 0, KVC_ERR_INVALID_ARG,
              "indptr[0] must be 0");
  int32_t num_empty = 0;
  for (int b = 0; b < batch; ++b) {
    KVC_REQUIRE(indptr_host[b + 1] >= indptr_host[b], KVC_ERR_INVALID_ARG,
                "indptr must be non-decreasing");
    num_empty += indptr_host[b + 1] == indptr_host[b];
  }
  const int64_t total = batch > 0 ? indptr_host[batch] : 0;
  const int hpw = heads_per_workgroup(group, head_dim, num_kv_heads);
  const int head_groups = (num_kv_heads + hpw - 1) / hpw;

  // Segments per KV-head group: one resident workgroup each, at most
  // kMaxSegPages pages each, at least one page each.  When the page cap
  // forces more segments than there are resident slots, the count is rounded
  // up to whole rounds of slots, so no round runs a few stragglers alone.
  int64_t segs = 0;
  if (total > 0) {
    const int64_t at_least = (total + kMaxSegPages - 1) / kMaxSegPages;
    if (num_segments_hint > 0) {
      segs = std::max<int64_t>(num_segments_hint, at_least);
    } else {
      const int64_t slots = int64_t(num_cus > 0 ? num_cus : 256) *
                            resident_workgroups_per_cu(group, head_dim, hpw);
      const int64_t per_round = (slots + head_groups - 1) / head_groups;
      segs = (std::max(per_round, at_least) + per_round - 1) / per_round * per_round;
    }
    segs = std::min<int64_t>(segs, total);
  }
  KVC_REQUIRE(segs <= (int64_t(1) << 30), KVC_ERR_INVALID_ARG, "too many segments");

  const std::vector<int64_t> cut = cut_segments(indptr_host, batch, total, segs);

  // Small batches (head_dim 128, no forced segment count): when every request
  // fits in kSmallMaxPages pages and the segments would cut a request,
  // one workgroup per (request, KV head) streams it and merges its waves'
  // states in LDS instead (no partials, no merge launch).
  int64_t max_pages = 0;
  for (int b = 0; b < batch; ++b)
    max_pages = std::max<int64_t>(max_pages, indptr_host[b + 1] - indptr_host[b]);
  bool splits = false;
  for (int64_t s = 1, bb = 0; s < segs && !splits; ++s) {
    const int64_t g = cut[size_t(s)];  // first page of segment s
    while (bb < batch && indptr_host[bb + 1] <= g) ++bb;
    splits = bb < batch && indptr_host[bb] < g;  // pages g-1 and g in request bb
  }
  if (num_segments_hint <= 0 && head_dim == 128 && total > 0 && max_pages <= kSmallMaxPages &&
      splits) {
    const int64_t need = kvc_decode_plan_ints(batch, batch);
    sched->batch = batch;
    sched->num_qo_heads = num_qo_heads;
    sched->num_kv_heads = num_kv_heads;
    sched->head_dim = head_dim;
    sched->page_size = page_size;
    sched->num_segments = batch;
    sched->num_head_groups = num_kv_heads;
    sched->heads_per_group = 1;
    sched->total_pages = int32_t(total);
    sched->num_empty = num_empty;
    sched->plan_ints = need;
    sched->small_batch = 1;
    KVC_REQUIRE(plan_host && plan_capacity >= need, KVC_ERR_WORKSPACE,
                "plan buffer too small: need " + std::to_string(need) + " int32");
    // One segment and one piece per request, empty requests included.
    int32_t* segments = plan_host;
    int32_t* pieces = plan_host + 4 * int64_t(batch);
    int32_t* nparts = pieces + 8 * (2 * int64_t(batch));
    for (int b = 0; b < batch; ++b) {
      const int32_t p0 = indptr_host[b], p1 = indptr_host[b + 1];
      int32_t* rec = segments + 4 * b;
      rec[0] = b;
      rec[1] = b + 1;
      rec[2] = p0;
      rec[3] = p1 - p0;
      int32_t* pc = pieces + 8 * b;
      pc[0] = b;
      pc[1] = p0;
      pc[2] = p1;
      pc[3] = -1;
      pc[4] = p1 - 1;
      pc[5] = last_page_len_host[b];
      pc[6] = 0;
      pc[7] = 0;
      nparts[b] = p1 > p0 ? 1 : 0;
    }
    sched->num_pieces = batch;
    sched->pieces_offset = 4 * batch;
    sched->nparts_offset = 4 * batch + 16 * batch;
    sched->max_partitions = 1;
    sched->workspace_bytes = 0;
    sched->append_pieces = 1;
    return ok();
  }

  const int64_t need = kvc_decode_plan_ints(batch, int32_t(segs));
  sched->batch = batch;
  sched->num_qo_heads = num_qo_heads;
  sched->num_kv_heads = num_kv_heads;
  sched->head_dim = head_dim;
  sched->page_size = page_size;
  sched->num_segments = int32_t(segs);
  sched->num_head_groups = head_groups;
  sched->heads_per_group = hpw;
  sched->total_pages = int32_t(total);
  sched->num_empty = num_empty;
  sched->plan_ints = need;
  sched->small_batch = 0;
  KVC_REQUIRE(plan_host && plan_capacity >= need, KVC_ERR_WORKSPACE,
              "plan buffer too small: need " + std::to_string(need) + " int32");

  // Plan image: segments [segs][4], pieces [num_pieces][8], req_nparts [batch].
  int32_t* segments = plan_host;
  const int64_t pieces_off = 4 * segs;
  int32_t* pieces = plan_host + pieces_off;
  int32_t* nparts = pieces + 8 * (segs + batch);
  std::fill(nparts, nparts + batch, 0);
  int64_t np = 0;
  int b = 0;
  int32_t append_pieces = 0;
  for (int64_t s = 0; s < segs; ++s) {
    const int64_t g0 = cut[size_t(s)];
    const int64_t g1 = cut[size_t(s) + 1];
    int32_t* rec = segments + 4 * s;
    rec[0] = int32_t(np);
    rec[2] = int32_t(g0);
    rec[3] = int32_t(g1 - g0);
    while (b < batch && indptr_host[b + 1] <= g0) ++b;
    for (int bb = b; bb < batch && indptr_host[bb] < g1; ++bb) {
      const int64_t sb = std::max<int64_t>(g0, indptr_host[bb]);
      const int64_t se = std::min<int64_t>(g1, indptr_host[bb + 1]);
      if (se > sb) {
        int32_t* pc = pieces + 8 * np++;
        pc[0] = bb;
        pc[1] = int32_t(sb);
        pc[2] = int32_t(se);
        pc[3] = nparts[bb]++;
        pc[4] = indptr_host[bb + 1] - 1;
        pc[5] = last_page_len_host ? last_page_len_host[bb] : kPage;
        pc[6] = 0;
        pc[7] = 0;
        // a request ending here: the fused append stages its new row by the
        // piece's index within the segment
        if (se == indptr_host[bb + 1])
          append_pieces = std::max<int32_t>(append_pieces, int32_t(np - rec[0]));
      }
    }
    rec[1] = int32_t(np);
  }
  int32_t max_parts = 1;
  for (int i = 0; i < batch; ++i) max_parts = std::max(max_parts, nparts[i]);
  // A request covered by a single piece is written directly (index -1).
  for (int64_t i = 0; i < np; ++i)
    if (nparts[pieces[8 * i]] == 1) pieces[8 * i + 3] = -1;
  sched->num_pieces = int32_t(np);
  sched->pieces_offset = int32_t(pieces_off);
  sched->nparts_offset = int32_t(pieces_off + 8 * (segs + batch));
  sched->max_partitions = max_parts;
  sched->workspace_bytes =
      kvc_decode_workspace_bytes(batch, num_qo_heads, head_dim, max_parts);
  sched->append_pieces = append_pieces;
  return ok();
}

namespace {
int decode_run(const kvc_decode_schedule* sched, const int32_t* plan, const void* q,
               int64_t q_batch_stride, const void* key_cache, const void* value_cache,
               int64_t cache_block_stride, int64_t cache_token_stride, int64_t num_blocks,
               const int32_t* indptr, const int32_t* indices, int64_t num_indices,
               const int32_t* last_page_len, const void* new_key, int64_t new_key_stride,
               const void* new_value, int64_t new_value_stride, float sm_scale,
               void* workspace, int64_t workspace_bytes, void* out, int64_t out_batch_stride,
               float* lse, void* stream) {
  KVC_REQUIRE(sched, KVC_ERR_INVALID_ARG, "null schedule");
  const int batch = sched->batch;
  if (batch == 0) return ok();
  // indices may be null (an empty tensor) when no request has a page; the
  // device indptr / last_page_len are not read (the plan image carries both).
  KVC_REQUIRE(plan && q && key_cache && value_cache && (indices || sched->total_pages == 0) &&
                  out,
              KVC_ERR_INVALID_ARG, "null pointer");
  const int Hq = sched->num_qo_heads, Hkv = sched->num_kv_heads, D = sched->head_dim;
  KVC_REQUIRE(Hkv > 0 && Hq % Hkv == 0, KVC_ERR_INVALID_ARG, "bad head counts");
  const int group = Hq / Hkv;
  KVC_REQUIRE(sched->page_size == kPage, KVC_ERR_UNSUPPORTED, "page_size must be 16");
  const bool small = sched->small_batch != 0;
  KVC_REQUIRE(sched->num_segments >= 0 && sched->max_partitions >= 1 &&
                  (small ? (D == 128 && sched->heads_per_group == 1 &&
                            sched->num_head_groups == Hkv && sched->num_segments == batch &&
                            sched->num_pieces == batch && sched->max_partitions == 1)
                         : (sched->heads_per_group == heads_per_workgroup(group, D, Hkv) &&
                            sched->num_head_groups ==
                                (Hkv + sched->heads_per_group - 1) / sched->heads_per_group)) &&
                  sched->plan_ints == kvc_decode_plan_ints(batch, sched->num_segments),
              KVC_ERR_INVALID_ARG, "schedule not produced by kvc_decode_plan");
  KVC_REQUIRE(num_blocks > 0 && num_indices >= sched->total_pages, KVC_ERR_INVALID_ARG,
              "bad num_blocks or fewer indices than planned pages");
  KVC_REQUIRE(cache_token_stride >= int64_t(Hkv) * D &&
                  cache_block_stride >= cache_token_stride * kPage,
              KVC_ERR_INVALID_ARG, "cache strides smaller than the block");
  KVC_REQUIRE(cache_token_stride * kPage * 2 < (int64_t(1) << 31), KVC_ERR_INVALID_ARG,
              "a cache block spans more than 2 GiB");
  KVC_REQUIRE(q_batch_stride >= int64_t(Hq) * D && out_batch_stride >= int64_t(Hq) * D,
              KVC_ERR_INVALID_ARG, "q/out batch stride smaller than Hq*head_dim");
  KVC_REQUIRE(sm_scale > 0.f, KVC_ERR_INVALID_ARG, "sm_scale must be positive");
  const int vec_bytes = D == 64 ? 8 : 16;
  KVC_REQUIRE(aligned(q, vec_bytes) && aligned(key_cache, vec_bytes) &&
                  aligned(value_cache, vec_bytes) &&
                  (q_batch_stride * 2) % vec_bytes == 0 &&
                  (cache_block_stride * 2) % vec_bytes == 0 &&
                  (cache_token_stride * 2) % vec_bytes == 0,
              KVC_ERR_ALIGNMENT, "q/cache pointers or strides not vector aligned");
  KVC_REQUIRE(aligned(out, 4) && out_batch_stride % 2 == 0 && aligned(plan, 16),
              KVC_ERR_ALIGNMENT, "out must be 4-byte aligned with an even batch stride, "
                                 "plan 16-byte aligned");
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
  a.indices = indices;
  a.num_indices = num_indices;
  a.segments = reinterpret_cast<const int4*>(plan);
  a.pieces = reinterpret_cast<const int4*>(plan + sched->pieces_offset);
  a.total_pages = sched->total_pages;
  a.num_segments = sched->num_segments;
  a.scale_log2 = sm_scale * kLog2e;
  a.num_kv_heads = Hkv;
  a.max_parts = sched->max_partitions;
  const int64_t rows = int64_t(batch) * Hq * sched->max_partitions;
  a.part_o = need ? static_cast<float*>(workspace) : nullptr;
  a.part_lse = need ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                              (rows * D * 4 + 255) / 256 * 256)
                    : nullptr;
  // Partials are written (streaming kernel) and read (merge) only for split
  // requests, which exist only when max_partitions > 1; with one piece per
  // request both kernels get null partials and never touch them.
  KVC_REQUIRE(sched->max_partitions == 1 || (a.part_o && a.part_lse), KVC_ERR_WORKSPACE,
              "a plan with split requests needs the partials workspace");
  a.out = static_cast<uint16_t*>(out);
  a.out_stride = out_batch_stride;
  a.lse = lse;
  a.new_k = static_cast<const uint16_t*>(new_key);
  a.new_v = static_cast<const uint16_t*>(new_value);
  a.new_k_stride = new_key_stride;
  a.new_v_stride = new_value_stride;
  if (new_key || new_value) {
    KVC_REQUIRE(new_key && new_value, KVC_ERR_INVALID_ARG, "new_key and new_value go together");
    KVC_REQUIRE(D == 128 &&
                    (small || (sched->heads_per_group == 8 && sched->append_pieces <= kNewMax)),
                KVC_ERR_UNSUPPORTED,
                "fused append needs head_dim 128 and either a small-batch schedule or a "
                "multiple of 8 KV heads with group <= 4 and at most " +
                    std::to_string(kNewMax) + " leading pieces per segment holding request "
                    "ends (schedule->append_pieces)");
    KVC_REQUIRE(new_key_stride >= int64_t(Hkv) * D && new_value_stride >= int64_t(Hkv) * D,
                KVC_ERR_INVALID_ARG, "new row stride smaller than a row");
    KVC_REQUIRE(aligned(new_key, 16) && aligned(new_value, 16) && new_key_stride % 8 == 0 &&
                    new_value_stride % 8 == 0,
                KVC_ERR_ALIGNMENT, "new rows must be 16-byte aligned");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (small) {
    // One workgroup per (request, KV head); outputs (empty requests too)
    // are written in the launch, no merge follows.
    const dim3 grid{unsigned(batch), unsigned(Hkv)};
    switch (group) {
      case 1: decode_small_kernel<1><<<grid, 64 * kSmallWaves, 0, s>>>(a); break;
      case 2: decode_small_kernel<2><<<grid, 64 * kSmallWaves, 0, s>>>(a); break;
      case 4: decode_small_kernel<4><<<grid, 64 * kSmallWaves, 0, s>>>(a); break;
      case 8: decode_small_kernel<8><<<grid, 64 * kSmallWaves, 0, s>>>(a); break;
      default:
        return set_error(KVC_ERR_UNSUPPORTED, "decode_run: unsupported group size " +
                                                  std::to_string(group));
    }
    KVC_LAUNCH_CHECK();
    return ok();
  }

  if (sched->num_segments > 0) {
    bool launched = false;
    const int segs = sched->num_segments, hg = sched->num_head_groups;
    const int hpw = sched->heads_per_group;
    if (D == 128) launched = dispatch_group<128>(group, a, segs, hg, hpw, s);
    else if (D == 64) launched = dispatch_group<64>(group, a, segs, hg, hpw, s);
    else if (D == 256) launched = dispatch_group<256>(group, a, segs, hg, hpw, s);
    KVC_REQUIRE(launched, KVC_ERR_UNSUPPORTED,
                "unsupported (group, head_dim) = (" + std::to_string(group) + ", " +
                    std::to_string(D) + ")");
    KVC_LAUNCH_CHECK();
  }
  // Single-piece requests were written by the streaming kernel; the merge
  // pass is needed for split requests and to zero empty ones.
  if (sched->max_partitions == 1 && sched->num_empty == 0) return ok();

  MergeArgs m;
  m.part_o = a.part_o;
  m.part_lse = a.part_lse;
  m.req_nparts = plan + sched->nparts_offset;
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

}  // namespace

extern "C" int kvc_batch_decode_run(
    const kvc_decode_schedule* sched, const int32_t* plan, const void* q,
    int64_t q_batch_stride, const void* key_cache, const void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride, int64_t num_blocks,
    const int32_t* indptr, const int32_t* indices, int64_t num_indices,
    const int32_t* last_page_len, float sm_scale, void* workspace,
    int64_t workspace_bytes, void* out, int64_t out_batch_stride, float* lse,
    void* stream) {
  return decode_run(sched, plan, q, q_batch_stride, key_cache, value_cache, cache_block_stride,
                    cache_token_stride, num_blocks, indptr, indices, num_indices, last_page_len,
                    nullptr, 0, nullptr, 0, sm_scale, workspace, workspace_bytes, out,
                    out_batch_stride, lse, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free decode run: the split-K partials live in this library's own
// device array instead of a caller workspace.  Each GPU the library runs on
// holds one copy of the array until the process ends; all calls on one GPU
// share it (calls that overlap on one GPU race on it).  The partials are
// written before they are read within a call, so nothing needs clearing.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[KVC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device`, which must be the current device:
// looked up once per device (hipGetSymbolAddress; the array's host-side name
// is not a device address and is never passed to a kernel or a copy).
int scratch_address(int device, void** out) {
  KVC_REQUIRE(device >= 0 && device < kMaxDevices, KVC_ERR_INVALID_ARG,
              "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    KVC_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    KVC_REQUIRE(p != nullptr, KVC_ERR_HIP, "hipGetSymbolAddress gave a null address");
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return ok();
}

}  // namespace

extern "C" int kvc_batch_decode_run_noalloc(
    const kvc_decode_schedule* sched, const int32_t* plan, const void* q,
    int64_t q_batch_stride, const void* key_cache, const void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride, int64_t num_blocks,
    const int32_t* indptr, const int32_t* indices, int64_t num_indices,
    const int32_t* last_page_len, float sm_scale, void* out, int64_t out_batch_stride,
    float* lse, void* stream) {
  KVC_REQUIRE(sched, KVC_ERR_INVALID_ARG, "null schedule");
  if (sched->batch == 0) return ok();
  const int64_t need =
      kvc_decode_workspace_bytes(sched->batch, sched->num_qo_heads, sched->head_dim,
                                 sched->max_partitions);
  KVC_REQUIRE(need <= KVC_NOALLOC_SCRATCH_BYTES, KVC_ERR_WORKSPACE,
              "the batch needs " + std::to_string(need) +
                  " bytes of split-K partials; the allocation-free run holds at most " +
                  std::to_string(int64_t(KVC_NOALLOC_SCRATCH_BYTES)) +
                  " (use kvc_batch_decode_run with a workspace)");
  int device = -1;
  KVC_HIP_CHECK(hipGetDevice(&device));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (s) {
    hipDevice_t sdev = -1;
    KVC_HIP_CHECK(hipStreamGetDevice(s, &sdev));
    KVC_REQUIRE(int(sdev) == device, KVC_ERR_INVALID_ARG,
                "the stream belongs to device " + std::to_string(int(sdev)) +
                    ", the current device is " + std::to_string(device));
  }
  void* ws = nullptr;
  const int st = scratch_address(device, &ws);
  if (st != KVC_OK) return st;
  return decode_run(sched, plan, q, q_batch_stride, key_cache, value_cache, cache_block_stride,
                    cache_token_stride, num_blocks, indptr, indices, num_indices, last_page_len,
                    nullptr, 0, nullptr, 0, sm_scale, ws, KVC_NOALLOC_SCRATCH_BYTES, out,
                    out_batch_stride, lse, stream);
}

extern "C" int kvc_batch_decode_append_run(
    const kvc_decode_schedule* sched, const int32_t* plan, const void* q,
    int64_t q_batch_stride, void* key_cache, void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride, int64_t num_blocks,
    const int32_t* indptr, const int32_t* indices, int64_t num_indices,
    const int32_t* last_page_len, const void* new_key, int64_t new_key_stride,
    const void* new_value, int64_t new_value_stride, float sm_scale, void* workspace,
    int64_t workspace_bytes, void* out, int64_t out_batch_stride, float* lse,
    void* stream) {
  KVC_REQUIRE(new_key && new_value, KVC_ERR_INVALID_ARG, "null new_key or new_value");
  return decode_run(sched, plan, q, q_batch_stride, key_cache, value_cache, cache_block_stride,
                    cache_token_stride, num_blocks, indptr, indices, num_indices, last_page_len,
                    new_key, new_key_stride, new_value, new_value_stride, sm_scale, workspace,
                    workspace_bytes, out, out_batch_stride, lse, stream);
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
