// Paged-KV prefill attention for gfx950 (MFMA): the queries of a chunk attend,
// causally, over everything the request has in the paged cache (the chunk's
// own tokens were appended before the call).  FlashInfer's
// BatchPrefillWithPagedKVCacheWrapper as the MoE engine uses it for
// continuation prefills (src/MoE/moe_engine.py:1733-1751, 3710-3727,
// 3939-3941).
//
// Work item = (request, tile of kTileRows query rows) x one KV head.  A query
// row is a (token, query head) pair: the `group` query heads that share a KV
// head are packed into the rows of one tile, so every K/V tile staged in LDS
// serves all of them (GQA reuse).  The four waves of a workgroup own 32 rows
// each; the workgroup walks the request's keys in tiles of 64.
//
// Per key tile, per wave, with v_mfma_f32_32x32x16_bf16 (A: lane l = row l%32,
// k = 8(l/32)..+7; B: lane l = column l%32, same k; C: acc[4i+j] = row
// 8i+4(l/32)+j, column l%32):
//   S^T = K Q^T   (keys x query rows): 2 key blocks x 8 k-steps of head dims;
//                 a lane ends up owning ONE query row (column l%32) and 32 of
//                 the tile's 64 keys, the other 32 being in lane l^32;
//   online softmax per lane (row), one exchange with lane l^32 for the row
//                 max and sum; the lane's P values are already laid out as
//                 the B operand of the next product (see the key order below);
//   O^T += V^T P^T  (head dims x query rows): 4 dim blocks x 4 k-steps of 16
//                 keys; O^T's columns are query rows too, so the per-row
//                 rescale by exp2(m_old - m_new) is a per-lane multiply.
// Key order inside a 16-key k-step: lane half h supplies k = 8h..8h+7, which
// the S^T accumulator layout gives as keys {4h..4h+3, 8+4h..8+4h+3}.  V^T is
// therefore stored in LDS with its 4-key groups 1 and 2 of every 16 swapped,
// so each lane's 8 keys are one 16-byte read.
//
// Staging: K as [key][dim] rows padded to 272 B (the q.k reads of 32 rows hit
// distinct banks), V transposed to [dim][key] rows padded to 144 B; each thread
// packs 4 keys x 8 dims with v_perm and writes 8-byte runs.  Two LDS tile
// buffers: tile t+1 is loaded into registers while tile t is computed, one
// barrier per tile.  Rows past the end of the cache are staged as zeros, so a
// masked key contributes exactly 0 (even if the page holds NaN bits).
#include "kvc_common.h"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <vector>

namespace kvc {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kWaveRows = 32;                 // query rows per wave
constexpr int kTileRows = 4 * kWaveRows;      // query rows per workgroup
constexpr int kKeys = 64;                     // keys per tile
constexpr int kPage = 16;
constexpr int kD = 128;
constexpr int kKPitch = kD * 2 + 16;          // bytes per K row in LDS
constexpr int kVPitch = kKeys * 2 + 16;       // bytes per V^T row in LDS
constexpr int kItemInts = 8;
constexpr float kRescaleLog2 = 8.f;           // lazy-rescale threshold (base 2)
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_stride;        // elements between query tokens
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t block_stride;    // elements between cache blocks
  int64_t token_stride;    // elements between tokens of a block
  int64_t num_blocks;
  const int32_t* indices;
  int64_t num_indices;
  const int4* items;       // [N][2]: (request, first query, q_len, kv_len),
                           //         (q offset, page offset, key tiles, pages)
  int32_t num_kv_heads;
  int32_t causal;
  float scale_log2;        // sm_scale * log2(e)
  uint16_t* out;
  int64_t out_stride;      // elements between output tokens
  float* lse;              // [total_q][Hq] natural log, may be null
};

struct alignas(16) TileBuf {
  uint8_t k[kKeys * kKPitch];
  uint8_t vt[kD * kVPitch];
};

// Position of key `k` (0..63) of a tile inside its V^T row: 4-key groups 1
// and 2 of every 16 are swapped.
__device__ __forceinline__ int vt_pos(int k) {
  const int grp = (k >> 2) & 3;
  const int sw = grp == 1 ? 2 : grp == 2 ? 1 : grp;
  return (k & ~15) | (sw << 2) | (k & 3);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Two floats as a bf16 pair (v_cvt_pk_bf16_f32: round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Two waves per SIMD (<= 256 VGPRs, no AGPRs): with one, the LDS-read and
// softmax latencies of a wave are exposed (262 -> 443 TFLOP/s measured on an
// 8 x 2048-token causal batch).  The softmax is the other limit -- the VALU
// runs beside the MFMAs of the other wave -- so it is kept lean: per-key
// tests only on boundary tiles, the scale folded into one FMA per score, the
// O rescale skipped unless a row max grows by more than 2^8, and P packed to
// bf16 with v_cvt_pk_bf16_f32 (443 -> 575 TFLOP/s on the same batch).
template <int G>
__global__ __launch_bounds__(kThreads, 2) void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int kTokPerWave = kWaveRows / G;
  __shared__ TileBuf tiles[2];

  const int h = blockIdx.y;
  const int4 it0 = a.items[2 * blockIdx.x];
  const int4 it1 = a.items[2 * blockIdx.x + 1];
  const int tok0 = it0.y, q_len = it0.z, kv_len = it0.w;
  const int q_off = it1.x, page_off = it1.y, ntiles = it1.z, npages = it1.w;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 31;
  const int half = lane >> 5;
  const int g = r % G;
  const int tok = tok0 + wave * kTokPerWave + r / G;
  const bool row_ok = tok < q_len;
  // Last key this row may see (inclusive).
  const int limit = !row_ok ? -1 : a.causal ? min(tok + kv_len - q_len, kv_len - 1) : kv_len - 1;
  const int hq = h * G + g;
  const int Hq = a.num_kv_heads * G;

  // Q as the B operand of S^T = K Q^T: k-step ks covers head dims
  // 16ks .. 16ks+15, lane half h the dims 16ks + 8h .. +7.
  bf16x8_t qb[kD / 16];
  {
    const int t = row_ok ? tok : 0;
    const uint16_t* qp = a.q + int64_t(q_off + t) * a.q_stride + int64_t(hq) * kD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks) {
      const uint4 v = row_ok ? *reinterpret_cast<const uint4*>(qp + 16 * ks) : make_uint4(0, 0, 0, 0);
      qb[ks] = as_bf16x8(v);
    }
  }

  // Staging roles.  K: thread t copies 16-byte chunk t%16 of token t/16 of
  // each of the tile's 4 pages.  V: thread t copies chunk t/16 of tokens
  // 4(t%16 % 4) .. +3 of page (t%16)/4 -- four consecutive keys, so that it
  // can write them transposed as 8-byte runs.
  const int t = threadIdx.x;
  const int k_tok = t >> 4, k_chunk = t & 15;
  const int v_grp = t & 15, v_chunk = t >> 4;
  const int v_page = v_grp >> 2, v_tok = (v_grp & 3) * 4;
  const int64_t head_off = int64_t(h) * kD;
  const char* kbase = reinterpret_cast<const char*>(a.k_cache);
  const char* vbase = reinterpret_cast<const char*>(a.v_cache);
  const int64_t blk_bytes = a.block_stride * 2;
  const int64_t tok_bytes = a.token_stride * 2;
  const uint32_t k_lane_off = uint32_t(k_tok * tok_bytes + (head_off + k_chunk * 8) * 2);

  uint4 kreg[4], vreg[4];
  // Page ids of a tile, fetched one iteration before its K/V loads need them
  // (four independent loads at clamped addresses; validity applied after),
  // so no load waits on an id.
  // Nothing reads the loaded ids until load_tile, so no wait sits here;
  // which of them exist is decided from the page index alone.
  struct TileIds { int32_t v[4]; int exists; };
  auto fetch_ids = [&](int tile) __attribute__((always_inline)) {
    TileIds t;
    t.exists = 0;
    const int64_t last = a.num_indices - 1;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = tile * 4 + u;
      t.v[u] = a.indices[min(int64_t(page_off) + p, last)];
      t.exists |= (p < npages && int64_t(page_off) + p <= last) ? (1 << u) : 0;
    }
    return t;
  };
  // load_tile returns a mask whose bit u says page u of the tile is real.
  auto load_tile = [&](const TileIds& t) __attribute__((always_inline)) {
    int ok = 0;
    int32_t ids[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int32_t id = __builtin_amdgcn_readfirstlane(t.v[u]);
      const bool good = ((t.exists >> u) & 1) && id >= 0 && id < a.num_blocks;
      ok |= good ? (1 << u) : 0;
      ids[u] = good ? id : 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const char* blk = kbase + int64_t(ids[u]) * blk_bytes;  // uniform
      kreg[u] = *reinterpret_cast<const uint4*>(blk + k_lane_off);
    }
    int32_t vid = ids[0];
#pragma unroll
    for (int u = 1; u < 4; ++u) vid = v_page == u ? ids[u] : vid;
    const char* vp = vbase + int64_t(vid) * blk_bytes + (head_off + v_chunk * 8) * 2;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      vreg[e] = *reinterpret_cast<const uint4*>(vp + (v_tok + e) * tok_bytes);
    return ok;
  };
  // Keys past the cache or in a missing page are staged as zeros: a mask
  // (v_and) on tiles that have such keys, nothing on the others.
  auto stage_tile = [&](TileBuf& buf, int tile, int ok) __attribute__((always_inline)) {
    const int key0 = tile * kKeys;
    if (ok != 0xF || key0 + kKeys > kv_len) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t m = (((ok >> u) & 1) && key0 + u * kPage + k_tok < kv_len) ? ~0u : 0u;
        kreg[u].x &= m; kreg[u].y &= m; kreg[u].z &= m; kreg[u].w &= m;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = v_page * kPage + v_tok + e;
        const uint32_t m = (((ok >> v_page) & 1) && key0 + key < kv_len) ? ~0u : 0u;
        vreg[e].x &= m; vreg[e].y &= m; vreg[e].z &= m; vreg[e].w &= m;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      *reinterpret_cast<uint4*>(buf.k + (u * kPage + k_tok) * kKPitch + k_chunk * 16) = kreg[u];
    // V: 8 dims x 4 keys written transposed.
    const uint32_t w[4][4] = {{vreg[0].x, vreg[0].y, vreg[0].z, vreg[0].w},
                              {vreg[1].x, vreg[1].y, vreg[1].z, vreg[1].w},
                              {vreg[2].x, vreg[2].y, vreg[2].z, vreg[2].w},
                              {vreg[3].x, vreg[3].y, vreg[3].z, vreg[3].w}};
    const int key = v_page * kPage + v_tok;
    uint8_t* dst = buf.vt + (v_chunk * 8) * kVPitch + vt_pos(key) * 2;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      // dims 2c (low halves) and 2c+1 (high halves) of the chunk
      const uint32_t lo01 = __builtin_amdgcn_perm(w[1][c], w[0][c], 0x05040100u);
      const uint32_t lo23 = __builtin_amdgcn_perm(w[3][c], w[2][c], 0x05040100u);
      const uint32_t hi01 = __builtin_amdgcn_perm(w[1][c], w[0][c], 0x07060302u);
      const uint32_t hi23 = __builtin_amdgcn_perm(w[3][c], w[2][c], 0x07060302u);
      *reinterpret_cast<uint2*>(dst + (2 * c) * kVPitch) = make_uint2(lo01, lo23);
      *reinterpret_cast<uint2*>(dst + (2 * c + 1) * kVPitch) = make_uint2(hi01, hi23);
    }
  };

  f32x16_t o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float m_run = kNegBig, l_run = 0.f;

  // Accumulator entry e of key block kb holds key 32kb + 8(e/4) + 4half + e%4
  // of the tile, which lies in page 2kb + e/8 of the tile.  Interior tiles
  // (every key visible to every row of the workgroup, all pages present)
  // skip the per-key tests: compute<false>.
  auto compute = [&](const TileBuf& buf, int tile, int ok, auto masked) __attribute__((always_inline)) {
    constexpr bool kMasked = decltype(masked)::value;
    // S^T for key blocks 0 and 1 (keys 32kb .. 32kb+31 of the tile).
    f32x16_t s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
      const uint8_t* krow = buf.k + (32 * kb + r) * kKPitch + 16 * half;
#pragma unroll
      for (int ks = 0; ks < kD / 16; ++ks) {
        const bf16x8_t ka = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 32 * ks));
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qb[ks], s[kb], 0, 0, 0);
      }
    }
    // Key offset (within the lane's half of the tile) this row may still see.
    const int rel = limit - tile * kKeys - 4 * half;
    auto visible = [&](int kb, int e) __attribute__((always_inline)) {
      if constexpr (kMasked)
        return (32 * kb + 8 * (e >> 2) + (e & 3)) <= rel && ((ok >> (2 * kb + (e >> 3))) & 1);
      else
        return true;
    };
    // Row max of the raw scores (the scale is positive), over this lane's 32
    // keys and lane l^32's.
    float mx = kNegBig;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (visible(kb, e)) mx = fmaxf(mx, s[kb][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // The running max only moves when some row's max grew by more than
    // kRescaleLog2 (base-2 units); otherwise the stale max stays, p <= 2^8,
    // and the O rescale is skipped -- same result, 64 fewer multiplies.
    const float cand = fmaxf(m_run, mx * a.scale_log2);
    if (__builtin_amdgcn_ballot_w64(cand > m_run + kRescaleLog2) != 0) {
      const float alpha = fast_exp2(m_run - cand);
      m_run = cand;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
    }
    float sum = 0.f;
    uint32_t pw[2][8];  // P as bf16 pairs, in S^T accumulator order
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float p0 = visible(kb, e) ? fast_exp2(fmaf(s[kb][e], a.scale_log2, -m_run)) : 0.f;
        const float p1 =
            visible(kb, e + 1) ? fast_exp2(fmaf(s[kb][e + 1], a.scale_log2, -m_run)) : 0.f;
        sum += p0 + p1;
        pw[kb][e >> 1] = pack_bf16(p0, p1);
      }
    sum += __shfl_xor(sum, 32);
    l_run += sum;
    // O^T += V^T P^T, k-step st = keys 16st .. 16st+15 of the tile, whose
    // P^T operand is accumulator entries 8(st%2) .. +7 of key block st/2.
#pragma unroll
    for (int st = 0; st < kKeys / 16; ++st) {
      const uint32_t* pp = &pw[st >> 1][4 * (st & 1)];
      const bf16x8_t pb = as_bf16x8(make_uint4(pp[0], pp[1], pp[2], pp[3]));
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8_t va = as_bf16x8(*reinterpret_cast<const uint4*>(
            buf.vt + (32 * db + r) * kVPitch + (16 * st + 8 * half) * 2));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, o[db], 0, 0, 0);
      }
    }
  };

  // Tiles [0, n_full) are interior for every row of the workgroup: all its
  // rows see keys up to at least lim_lo (its first token's limit), and a
  // first pass checks that every page the item visits exists.
  int bad = 0;
  const int pages_used = min(npages, ntiles * 4);
  for (int p = threadIdx.x; p < pages_used; p += kThreads) {
    const int64_t at = int64_t(page_off) + p;
    const int32_t id = at < a.num_indices ? a.indices[at] : -1;
    bad |= id < 0 || id >= a.num_blocks;
  }
  const bool all_pages = __syncthreads_and(bad == 0);
  const int lim_lo = a.causal ? tok0 + kv_len - q_len : kv_len - 1;
  const int n_full = all_pages ? max(0, min(ntiles, (lim_lo + 1) / kKeys)) : 0;
  // Per iteration: K/V loads of tile+1 (ids fetched last iteration), id
  // fetch of tile+2, the tile's math, staging of tile+1, one barrier.
  TileIds ids_next;
  auto run_tiles = [&](int t0, int t1, int ok, auto masked) __attribute__((always_inline)) {
    for (int tile = t0; tile < t1; ++tile) {
      int next_ok = 0;
      if (tile + 1 < ntiles) {
        next_ok = load_tile(ids_next);
        if (tile + 2 < ntiles) ids_next = fetch_ids(tile + 2);
      }
      compute(tiles[tile & 1], tile, ok, masked);
      if (tile + 1 < ntiles) stage_tile(tiles[(tile + 1) & 1], tile + 1, next_ok);
      ok = next_ok;
      __syncthreads();
    }
    return ok;
  };
  if (ntiles > 0) {
    int ok = load_tile(fetch_ids(0));
    if (ntiles > 1) ids_next = fetch_ids(1);
    stage_tile(tiles[0], 0, ok);
    __syncthreads();
    ok = run_tiles(0, n_full, ok, std::false_type{});
    run_tiles(n_full, ntiles, ok, std::true_type{});
  }

  if (!row_ok) return;
  // O^T column r = this row; entry (db, 4i+j) = head dim 32db + 8i + 4half + j.
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  uint16_t* dst = a.out + int64_t(q_off + tok) * a.out_stride + int64_t(hq) * kD + 4 * half;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<uint2*>(dst + 32 * db + 8 * i) =
          make_uint2(pack_bf16(o[db][4 * i] * inv, o[db][4 * i + 1] * inv),
                     pack_bf16(o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv));
    }
  if (a.lse && half == 0)
    a.lse[int64_t(q_off + tok) * Hq + hq] = l_run > 0.f ? (m_run + fast_log2(l_run)) * kLn2 : -INFINITY;
}

template <int G>
void launch(const PrefillArgs& a, int items, int hkv, hipStream_t s) {
  prefill_mfma_kernel<G><<<dim3(unsigned(items), unsigned(hkv)), kThreads, 0, s>>>(a);
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_prefill_plan(const int32_t* qo_indptr_host, const int32_t* kv_indptr_host,
                                const int32_t* last_page_len_host, int32_t batch,
                                int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t page_size, int32_t causal,
                                kvc_prefill_schedule* sched, int32_t* plan_host,
                                int64_t plan_capacity) {
  KVC_REQUIRE(sched, KVC_ERR_INVALID_ARG, "null schedule");
  KVC_REQUIRE(batch >= 0, KVC_ERR_INVALID_ARG, "negative batch");
  KVC_REQUIRE(batch == 0 || (qo_indptr_host && kv_indptr_host && last_page_len_host),
              KVC_ERR_INVALID_ARG, "null indptr / last_page_len");
  KVC_REQUIRE(num_kv_heads > 0 && num_qo_heads > 0 && num_qo_heads % num_kv_heads == 0,
              KVC_ERR_INVALID_ARG, "num_qo_heads must be a positive multiple of num_kv_heads");
  const int group = num_qo_heads / num_kv_heads;
  KVC_REQUIRE(head_dim == kD && page_size == kPage &&
                  (group == 1 || group == 2 || group == 4 || group == 8),
              KVC_ERR_UNSUPPORTED,
              "prefill supports head_dim 128, page_size 16, group 1/2/4/8");
  const int tile_tokens = kTileRows / group;
  std::vector<int32_t> rec;
  int64_t total_q = 0;
  int max_tiles = 0;
  for (int b = 0; b < batch; ++b) {
    const int64_t q_len = int64_t(qo_indptr_host[b + 1]) - qo_indptr_host[b];
    const int64_t pages = int64_t(kv_indptr_host[b + 1]) - kv_indptr_host[b];
    KVC_REQUIRE(q_len >= 0 && pages >= 0, KVC_ERR_INVALID_ARG,
                "qo_indptr and kv_indptr must be non-decreasing");
    const int lpl = last_page_len_host[b];
    KVC_REQUIRE(pages == 0 || (lpl >= 1 && lpl <= kPage), KVC_ERR_INVALID_ARG,
                "last_page_len must be in 1..page_size for a request with pages");
    const int64_t kv_len = pages > 0 ? (pages - 1) * kPage + lpl : 0;
    KVC_REQUIRE(kv_len < (int64_t(1) << 30) && q_len < (int64_t(1) << 30), KVC_ERR_INVALID_ARG,
                "request too long");
    total_q += q_len;
    for (int64_t t0 = 0; t0 < q_len; t0 += tile_tokens) {
      const int64_t last = std::min<int64_t>(t0 + tile_tokens, q_len) - 1;
      int64_t keys = causal ? last + kv_len - q_len + 1 : kv_len;
      keys = std::max<int64_t>(0, std::min<int64_t>(keys, kv_len));
      const int tiles = int((keys + kKeys - 1) / kKeys);
      max_tiles = std::max(max_tiles, tiles);
      const int32_t r8[kItemInts] = {b, int32_t(t0), int32_t(q_len), int32_t(kv_len),
                                     qo_indptr_host[b], kv_indptr_host[b], tiles, int32_t(pages)};
      rec.insert(rec.end(), r8, r8 + kItemInts);
    }
  }
  const int64_t n = int64_t(rec.size()) / kItemInts;
  KVC_REQUIRE(n < (int64_t(1) << 31), KVC_ERR_INVALID_ARG, "too many query tiles");
  sched->batch = batch;
  sched->num_qo_heads = num_qo_heads;
  sched->num_kv_heads = num_kv_heads;
  sched->head_dim = head_dim;
  sched->page_size = page_size;
  sched->causal = causal ? 1 : 0;
  sched->tile_tokens = tile_tokens;
  sched->num_items = int32_t(n);
  sched->total_q = int32_t(std::min<int64_t>(total_q, INT32_MAX));
  sched->max_key_tiles = max_tiles;
  sched->plan_ints = n * kItemInts;
  KVC_REQUIRE(plan_host && plan_capacity >= sched->plan_ints, KVC_ERR_WORKSPACE,
              "plan buffer too small: need " + std::to_string(sched->plan_ints) + " int32");
  // Longest items first: the causal tail of short tiles fills the gaps.
  std::vector<int64_t> order(n);
  for (int64_t i = 0; i < n; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int64_t x, int64_t y) {
    return rec[x * kItemInts + 6] > rec[y * kItemInts + 6];
  });
  for (int64_t i = 0; i < n; ++i)
    std::copy_n(rec.data() + order[i] * kItemInts, kItemInts, plan_host + i * kItemInts);
  return ok();
}

extern "C" int kvc_batch_prefill_run(const kvc_prefill_schedule* sched, const int32_t* plan,
                                     const void* q, int64_t q_token_stride,
                                     const void* key_cache, const void* value_cache,
                                     int64_t cache_block_stride, int64_t cache_token_stride,
                                     int64_t num_blocks, const int32_t* indices,
                                     int64_t num_indices, float sm_scale, void* out,
                                     int64_t out_token_stride, float* lse, void* stream) {
  KVC_REQUIRE(sched, KVC_ERR_INVALID_ARG, "null schedule");
  const int Hq = sched->num_qo_heads, Hkv = sched->num_kv_heads;
  KVC_REQUIRE(Hkv > 0 && Hq % Hkv == 0 && sched->head_dim == kD && sched->page_size == kPage &&
                  sched->tile_tokens == kTileRows / (Hq / Hkv) &&
                  sched->plan_ints == int64_t(sched->num_items) * kItemInts,
              KVC_ERR_INVALID_ARG, "schedule not produced by kvc_prefill_plan");
  if (sched->num_items == 0) return ok();
  KVC_REQUIRE(plan && q && key_cache && value_cache && out && indices, KVC_ERR_INVALID_ARG,
              "null pointer");
  KVC_REQUIRE(num_blocks > 0 && num_indices > 0, KVC_ERR_INVALID_ARG,
              "bad num_blocks or empty indices");
  KVC_REQUIRE(cache_token_stride >= int64_t(Hkv) * kD && cache_block_stride >= cache_token_stride * kPage,
              KVC_ERR_INVALID_ARG, "cache strides smaller than the block");
  KVC_REQUIRE(cache_token_stride * kPage * 2 < (int64_t(1) << 31), KVC_ERR_INVALID_ARG,
              "a cache block spans more than 2 GiB");
  KVC_REQUIRE(q_token_stride >= int64_t(Hq) * kD && out_token_stride >= int64_t(Hq) * kD,
              KVC_ERR_INVALID_ARG, "q/out token stride smaller than Hq*head_dim");
  KVC_REQUIRE(sm_scale > 0.f, KVC_ERR_INVALID_ARG, "sm_scale must be positive");
  KVC_REQUIRE(aligned(q, 16) && aligned(key_cache, 16) && aligned(value_cache, 16) &&
                  aligned(out, 8) && aligned(plan, 16) && q_token_stride % 8 == 0 &&
                  out_token_stride % 4 == 0 && cache_block_stride % 8 == 0 &&
                  cache_token_stride % 8 == 0,
              KVC_ERR_ALIGNMENT, "q/cache/plan must be 16-byte aligned (out 8-byte) with "
                                 "matching strides");
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_stride = q_token_stride;
  a.k_cache = static_cast<const uint16_t*>(key_cache);
  a.v_cache = static_cast<const uint16_t*>(value_cache);
  a.block_stride = cache_block_stride;
  a.token_stride = cache_token_stride;
  a.num_blocks = num_blocks;
  a.indices = indices;
  a.num_indices = num_indices;
  a.items = reinterpret_cast<const int4*>(plan);
  a.num_kv_heads = Hkv;
  a.causal = sched->causal;
  a.scale_log2 = sm_scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.out_stride = out_token_stride;
  a.lse = lse;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (Hq / Hkv) {
    case 1: launch<1>(a, sched->num_items, Hkv, s); break;
    case 2: launch<2>(a, sched->num_items, Hkv, s); break;
    case 4: launch<4>(a, sched->num_items, Hkv, s); break;
    case 8: launch<8>(a, sched->num_items, Hkv, s); break;
    default: KVC_REQUIRE(false, KVC_ERR_UNSUPPORTED, "group must be 1, 2, 4 or 8");
  }
  KVC_LAUNCH_CHECK();
  return ok();
}
