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
// kernels are HBM-bound and run on the VALU (no MFMA).  Work decomposition:
//   * grid (num_kv_heads, max_partitions, batch), KV head fastest: the
//     workgroups of the heads of one page range are dispatched together (to
//     the eight XCDs in turn), so the 2 KB token rows of a page are read by
//     concurrent workgroups, and every XCD receives the same share of work
//     whatever the spread of request lengths;
//   * a 256-thread workgroup owns one (request, KV head, partition of
//     pages_per_partition pages) and serves all `group` query heads of that KV
//     head, so K/V are read from HBM exactly once; wave w takes pages
//     p0 + w, p0 + w + 4, ...  Each wave's page ids are loaded once, one per
//     lane, and broadcast with v_readlane, so no dependent global load sits
//     in the streaming loop;
//   * epilogue: the four waves merge through LDS; a request with one partition
//     is written as bf16 directly, otherwise an fp32 partial + log2-sum-exp
//     goes to the workspace and decode_merge_kernel folds them.
//
// head_dim 128 (the reference models) uses decode_lds_kernel: each wave stages
// one page (16 tokens x 256 B of K and of V) from HBM through registers into
// its own 8 KB LDS tile while the previous page is being consumed.  The tile
// is stored with the 16-byte chunk c of token t at slot c ^ t, which makes
// both read patterns below free of LDS bank conflicts:
//   q.k : lane (token t, query head g) computes the whole 128-dim dot product
//         with v_dot2_f32_bf16 from 16 ds_read_b128 of row t (the four lanes
//         of a token read the same address); no cross-lane reduction;
//   p.v : lane l owns dims 2l, 2l+1 for every query head; per token one
//         ds_read_b32 of V and one broadcast read of p[t][0..G).
// Softmax statistics live per 16-lane DPP row (one query head per row).
// head_dim 64 and 256 use decode_reg_kernel, which keeps K/V in registers:
// lane (row r, column c) holds 16 B of tokens r, r+4, r+8, r+12 and q.k is
// reduced over the 16 lanes of a DPP row.
#include "kvc_common.h"

#include <algorithm>
#include <cmath>

namespace kvc {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPage = 16;      // tokens per page (the engine's page_size)
constexpr int kTokPerRow = 4;  // register kernel: tokens of a page per 16-lane row
constexpr int kMaxPagesPerPart = 4 * 64;  // a wave holds its page ids in 64 lanes
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

// Compiler-level ordering point for LDS traffic between lanes of one wave
// (the LDS unit itself executes one wave's instructions in order).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp<kDppRowRor4>(v));
  v = fmaxf(v, dpp<kDppRowRor8>(v));
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Page ids of the calling wave: lane j holds the block id of the wave's j-th
// page (page p0 + wave + 4j of the request), -1 past the end.
__device__ __forceinline__ int32_t load_wave_page_ids(const DecodeArgs& a, int pbeg,
                                                      int first, int nw, int lane) {
  int32_t id = -1;
  if (lane < nw) {
    const int64_t slot = int64_t(pbeg) + first + int64_t(kWaves) * lane;
    id = slot < a.num_indices ? a.indices[slot] : -1;
  }
  return id;
}

// Wave-merge + output.  s_acc [kWaves][G][D], s_m / s_l [kWaves][G] hold each
// wave's unnormalised accumulator and base-2 softmax statistics.
template <int G, int D>
__device__ __forceinline__ void finish_partition(const DecodeArgs& a, int b, int h, int part,
                                                 int nparts, const float* s_acc,
                                                 const float* s_m, const float* s_l) {
  const int hq0 = h * G;
  const int64_t part_base = (int64_t(b) * a.num_kv_heads + h) * a.max_parts + part;
  for (int o = threadIdx.x; o < G * D; o += kThreads) {
    const int g = o / D;
    const int d = o - g * D;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, s_m[w * G + g]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(s_m[w * G + g] - mm);
      L = fmaf(s_l[w * G + g], f, L);
      A = fmaf(s_acc[(w * G + g) * D + d], f, A);
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

struct __align__(16) PageTile {
  uint4 k[kPage * 16];  // [token][slot], slot = chunk ^ token
  uint4 v[kPage * 16];
  float p[kPage * 8];   // softmax weights p[token][query head], G <= 8
};

template <int G>
__global__ __launch_bounds__(kThreads) void decode_lds_kernel(DecodeArgs a) {
  using C = LdsCfg<G>;
  constexpr int D = 128;
  __shared__ PageTile s_tile[kWaves];
  static_assert(sizeof(s_tile) >= sizeof(float) * (kWaves * G * D + 2 * kWaves * G),
                "epilogue does not fit in the page tiles");

  const int h = blockIdx.x;
  const int part = blockIdx.y;
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
  PageTile& tile = s_tile[wave];

  // q.k role: token t, query head gq (and gq + 4 when G == 8), dim split.
  const int t = lane & 15;
  const int row = lane >> 4;
  const int gq = row % C::GP;
  const int split = row / C::GP;
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
  // Staging role: load instruction u moves tokens 4u..4u+3; lane -> (token, slot).
  const int st_tok = lane >> 4;
  const int st_slot = lane & 15;
  int32_t st_off[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int tok = 4 * u + st_tok;
    st_off[u] = int32_t(tok * a.token_stride) + h * D + ((st_slot ^ tok) << 3);
  }
  // p.v role: dims 2*lane, 2*lane+1 = word lane&3 of chunk lane>>2.
  const int vchunk = lane >> 2;
  const int vword = lane & 3;

  const int nw = p1 - p0 > wave ? (p1 - p0 - wave + kWaves - 1) / kWaves : 0;
  const int32_t my_ids = load_wave_page_ids(a, pbeg, p0 + wave, nw, lane);

  float m_run[C::QL], l_run[C::QL], acc[G][2];
#pragma unroll
  for (int ql = 0; ql < C::QL; ++ql) {
    m_run[ql] = kNegBig;
    l_run[ql] = 0.f;
  }
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;

  uint4 rk[4], rv[4];
  auto issue = [&](int32_t blk) {
    const int64_t base = int64_t(blk) * a.block_stride;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      rk[u] = *reinterpret_cast<const uint4*>(a.k_cache + base + st_off[u]);
      rv[u] = *reinterpret_cast<const uint4*>(a.v_cache + base + st_off[u]);
    }
  };
  auto safe_id = [&](int32_t id) { return (id >= 0 && id < a.num_blocks) ? id : 0; };

  int32_t blk = nw > 0 ? __builtin_amdgcn_readlane(my_ids, 0) : 0;
  if (nw > 0) issue(safe_id(blk));
  for (int j = 0; j < nw; ++j) {
    const int pi = p0 + wave + kWaves * j;
    const bool blk_ok = blk >= 0 && blk < a.num_blocks;
    const int valid = !blk_ok ? 0 : (pi == npages - 1 ? last_len : kPage);
    if (valid < kPage) {
      // Rows past the end may hold anything (even NaN bits): stage zeros so
      // that 0 * v stays 0.
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (4 * u + st_tok >= valid) rk[u] = rv[u] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      tile.k[u * 64 + lane] = rk[u];
      tile.v[u * 64 + lane] = rv[u];
    }
    if (j + 1 < nw) {
      blk = __builtin_amdgcn_readlane(my_ids, j + 1);
      issue(safe_id(blk));  // in flight while this page is consumed
    }
    wave_lds_fence();

    // q.k: lane (t, gq) over its chunks of K row t.
    float dots[C::QL];
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) dots[ql] = 0.f;
    const uint4* krow = tile.k + t * 16;
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const int c = split * C::CH + i;
      const uint4 kv = krow[c ^ t];
#pragma unroll
      for (int ql = 0; ql < C::QL; ++ql) {
        dots[ql] = dot2_bf16(qw[ql][4 * i + 0], kv.x, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * i + 1], kv.y, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * i + 2], kv.z, dots[ql]);
        dots[ql] = dot2_bf16(qw[ql][4 * i + 3], kv.w, dots[ql]);
      }
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
      if (row < C::GP) tile.p[t * G + gq + 4 * ql] = p;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float al = readlane_f(alpha[g / 4], 16 * (g % 4));
      acc[g][0] *= al;
      acc[g][1] *= al;
    }
    wave_lds_fence();

    // p.v over the 16 tokens of the page (rows past `valid` are zero).
    const char* vbase = reinterpret_cast<const char*>(tile.v) + vword * 4;
#pragma unroll
    for (int tt = 0; tt < kPage; ++tt) {
      const uint32_t vw =
          *reinterpret_cast<const uint32_t*>(vbase + tt * 256 + ((vchunk ^ tt) << 4));
      const float v0 = bf16lo(vw);
      const float v1 = bf16hi(vw);
      float pg[G];
      if constexpr (G >= 4) {
#pragma unroll
        for (int q4 = 0; q4 < G / 4; ++q4) {
          const float4 x = reinterpret_cast<const float4*>(tile.p + tt * G)[q4];
          pg[4 * q4 + 0] = x.x;
          pg[4 * q4 + 1] = x.y;
          pg[4 * q4 + 2] = x.z;
          pg[4 * q4 + 3] = x.w;
        }
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) pg[g] = tile.p[tt * G + g];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        acc[g][0] = fmaf(pg[g], v0, acc[g][0]);
        acc[g][1] = fmaf(pg[g], v1, acc[g][1]);
      }
    }
    wave_lds_fence();
  }

  // Workgroup epilogue (the page tiles are reused for the wave partials).
  __syncthreads();
  float* s_acc = reinterpret_cast<float*>(s_tile);
  float* s_m = s_acc + kWaves * G * D;
  float* s_l = s_m + kWaves * G;
#pragma unroll
  for (int g = 0; g < G; ++g)
    *reinterpret_cast<float2*>(s_acc + (wave * G + g) * D + 2 * lane) =
        make_float2(acc[g][0], acc[g][1]);
  if (t == 0 && row < C::GP) {
#pragma unroll
    for (int ql = 0; ql < C::QL; ++ql) {
      s_m[wave * G + gq + 4 * ql] = m_run[ql];
      s_l[wave * G + gq + 4 * ql] = l_run[ql];
    }
  }
  __syncthreads();
  finish_partition<G, D>(a, b, h, part, nparts, s_acc, s_m, s_l);
}

// ---------------------------------------------------------------------------
// head_dim 64 / 256: register kernel.
// ---------------------------------------------------------------------------
// Load the D/16 bf16 elements one lane owns (D/32 32-bit words).
template <int D>
__device__ __forceinline__ void load_slice(uint32_t (&w)[D / 32], const uint16_t* p) {
  if constexpr (D == 64) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    w[0] = x.x; w[1] = x.y;
  } else {
    static_assert(D == 128 || D == 256, "head_dim must be 64, 128 or 256");
#pragma unroll
    for (int i = 0; i < D / 128; ++i) {
      const uint4 x = reinterpret_cast<const uint4*>(p)[i];
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
    load_slice<D>(r.k[j], a.k_cache + base + int64_t(j) * kTokPerRow * a.token_stride);
#pragma unroll
  for (int j = 0; j < kTokPerRow; ++j)
    load_slice<D>(r.v[j], a.v_cache + base + int64_t(j) * kTokPerRow * a.token_stride);
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
  __shared__ float s_acc[kWaves * G * D];
  __shared__ float s_m[kWaves * G];
  __shared__ float s_l[kWaves * G];
  const int h = blockIdx.x;
  const int part = blockIdx.y;
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
  const int nw = p1 - p0 > wave ? (p1 - p0 - wave + kWaves - 1) / kWaves : 0;
  const int32_t my_ids = load_wave_page_ids(a, pbeg, p0 + wave, nw, lane);
  auto id_at = [&](int j) { return __builtin_amdgcn_readlane(my_ids, j); };
  auto safe = [&](int32_t id) { return (id >= 0 && id < a.num_blocks) ? id : 0; };
  auto valid_at = [&](int j, int32_t id) {
    if (id < 0 || id >= a.num_blocks) return 0;
    return p0 + wave + kWaves * j == npages - 1 ? last_len : kPage;
  };

  // Two register sets: page j is consumed while page j+1 is in flight.
  PageRegs<D> ra, rb;
  int32_t ida = 0, idb = 0;
  if (nw > 0) {
    ida = id_at(0);
    load_page_regs<D>(a, ra, safe(ida), lane_off);
  }
  for (int j = 0; j < nw; j += 2) {
    if (j + 1 < nw) {
      idb = id_at(j + 1);
      load_page_regs<D>(a, rb, safe(idb), lane_off);
    }
    consume_page_regs<G, D>(qw, ra, valid_at(j, ida), row, a.scale_log2, m, l, acc);
    if (j + 1 >= nw) break;
    if (j + 2 < nw) {
      ida = id_at(j + 2);
      load_page_regs<D>(a, ra, safe(ida), lane_off);
    }
    consume_page_regs<G, D>(qw, rb, valid_at(j + 1, idb), row, a.scale_log2, m, l, acc);
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
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < E; ++e) s_acc[(wave * G + g) * D + col * E + e] = acc[g][e];
      if (col == 0) {
        s_m[wave * G + g] = m[g];
        s_l[wave * G + g] = l[g];
      }
    }
  }
  __syncthreads();
  finish_partition<G, D>(a, b, h, part, nparts, s_acc, s_m, s_l);
}

// ---------------------------------------------------------------------------
// Split-K merge.
// ---------------------------------------------------------------------------
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

// One wave per (request, query head): lane p reads the log2-sum-exp of
// partition p, the wave forms the weights, then every lane folds its D/64
// dims over the partitions (independent loads, unrolled).  Requests with a
// single partition were finished by the partition kernel; requests with no
// pages get a zero output and lse = -inf.
template <int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(MergeArgs a) {
  constexpr int EPL = D / 64;  // dims per lane
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
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
  const float* lp = a.part_lse + base * G + g;  // partition p at lp[p * G]

  float mx = -INFINITY;
  for (int p = lane; p < nparts; p += 64) mx = fmaxf(mx, lp[int64_t(p) * G]);
  mx = wave_max(mx);
  if (nparts == 0 || mx == -INFINITY) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) out[lane * EPL + e] = 0;
    if (a.lse && lane == 0) a.lse[int64_t(b) * Hq + hq] = -INFINITY;
    return;
  }
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  float S = 0.f;
  for (int q0 = 0; q0 < nparts; q0 += 64) {
    const float w = q0 + lane < nparts ? fast_exp2(lp[int64_t(q0 + lane) * G] - mx) : 0.f;
    S += w;
    const int n = min(64, nparts - q0);
#pragma unroll 4
    for (int j = 0; j < n; ++j) {
      const float wj = readlane_f(w, j);
      const float* po = a.part_o + ((base + q0 + j) * G + g) * D + lane * EPL;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = fmaf(wj, po[e], acc[e]);
    }
  }
  S = wave_sum(S);
  const float inv = 1.f / S;
#pragma unroll
  for (int e = 0; e < EPL; ++e) out[lane * EPL + e] = f32_to_bf16(acc[e] * inv);
  if (a.lse && lane == 0) a.lse[int64_t(b) * Hq + hq] = (mx + fast_log2(S)) * kLn2;
}

template <int G, int D>
void launch_partition(const DecodeArgs& a, int batch, hipStream_t s) {
  const dim3 grid(unsigned(a.num_kv_heads), unsigned(a.max_parts), unsigned(batch));
  if constexpr (D == 128)
    decode_lds_kernel<G><<<grid, kThreads, 0, s>>>(a);
  else
    decode_reg_kernel<G, D><<<grid, kThreads, 0, s>>>(a);
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
    ppp = std::min((pages_per_partition_hint + 3) / 4 * 4, kMaxPagesPerPart);
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
                  sched->pages_per_partition <= kMaxPagesPerPart &&
                  sched->max_partitions >= 1 && sched->max_partitions <= 65535,
              KVC_ERR_INVALID_ARG, "schedule not produced by kvc_decode_plan");
  KVC_REQUIRE(num_blocks > 0 && num_indices >= 0, KVC_ERR_INVALID_ARG,
              "bad num_blocks / num_indices");
  KVC_REQUIRE(cache_token_stride >= int64_t(Hkv) * D &&
                  cache_block_stride >= cache_token_stride * kPage,
              KVC_ERR_INVALID_ARG, "cache strides smaller than the block");
  KVC_REQUIRE(cache_token_stride * kPage < (int64_t(1) << 31), KVC_ERR_INVALID_ARG,
              "a cache block spans more than 2^31 elements");
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
