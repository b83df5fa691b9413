// Paged-KV prefill attention for gfx950 (MFMA): the queries of a chunk attend,
// causally, over everything the request has in the paged cache (the chunk's
// own tokens were appended before the call).  FlashInfer's
// BatchPrefillWithPagedKVCacheWrapper as the MoE engine uses it for
// continuation prefills (src/MoE/moe_engine.py:1733-1751, 3710-3727,
// 3939-3941).
//
// Work unit = (request, tile of kTileRows query rows) x one KV head.  A query
// row is a (token, query head) pair: the `group` query heads that share a KV
// head are packed into the rows of one tile, so every K/V tile staged in LDS
// serves all of them (GQA reuse).  The eight waves of a workgroup own 32 rows
// each and walk the request's keys in tiles of 64.  At most one workgroup
// per CU is launched; each runs a list of units made by the host plan.
//
// Per key tile, per wave, with v_mfma_f32_32x32x16_bf16 (A: lane l = row l%32,
// k = 8(l/32)..+7; B: lane l = column l%32, same k; C: acc[4i+j] = row
// 8i+4(l/32)+j, column l%32):
//   S^T = K Q^T   (keys x query rows): 2 key blocks x 8 k-steps of head dims;
//                 a lane ends up owning ONE query row (column l%32) and 32 of
//                 the tile's 64 keys, the other 32 being in lane l^32;
//   online softmax per lane (row), one exchange with lane l^32 for the row
//                 max (the row sum stays split between the two lanes until
//                 the end); the lane's P values are already laid out as the
//                 B operand of the next product (see the key order below);
//   O^T += V^T P^T  (head dims x query rows): 4 dim blocks x 4 k-steps of 16
//                 keys; O^T's columns are query rows too, so the per-row
//                 rescale by exp2(m_old - m_new) is a per-lane multiply.
// Key order inside a 16-key k-step: lane half h supplies k = 8h..8h+7, which
// the S^T accumulator layout gives as keys {4h..4h+3, 8+4h..8+4h+3}; the V^T
// operand is read in that order.
//
// Staging: K and V go from memory straight into LDS (global_load_lds_dwordx4,
// buffer_load_dwordx4 ... lds) as unpadded [key][dim] rows whose 16-byte
// chunks are XOR-swizzled by key, so that the MFMA operand reads hit distinct
// banks: K as 16-byte reads of one key's dims, V^T through the transposing
// ds_read_b64_tr_b16.  Two LDS buffers per operand.  V rows past the end of
// the cache or in a missing page load as zeros (the buffer load is bounded to
// the page's valid tokens), so a masked key contributes exactly 0 even if the
// page holds NaN bits.  Each wave also has an LDS area of its own through
// which its finished rows leave as whole rows (128 KB of LDS in all, one
// workgroup per CU).
#include "kvc_common.h"

#include <algorithm>
#include <queue>
#include <cmath>
#include <type_traits>
#include <vector>

namespace kvc {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr int kThreads = 512;
constexpr int kWaveRows = 32;                 // query rows per wave
constexpr int kTileRows = 8 * kWaveRows;      // query rows per workgroup
constexpr int kKeys = 64;                     // keys per tile
constexpr int kPage = 16;
constexpr int kD = 128;
constexpr int kKRow = kD * 2;                // bytes per K or V row in LDS (unpadded)
constexpr int kORow = kKRow + 16;            // bytes per staged output row
constexpr int kItemInts = 8;
constexpr float kRescaleLog2 = 8.f;           // lazy-rescale threshold (base 2)
// Word 3 of a raw buffer resource (32-bit data, no swizzle): loads past
// num_records return zeros.
constexpr int kBufferRsrcWord3 = 0x00020000;
// s_waitcnt vmcnt(0) with the other counters unconstrained (gfx9 encoding:
// vmcnt [3:0],[15:14]; expcnt [6:4]; lgkmcnt [11:8]).
constexpr int kWaitVmcnt0 = 0x0F70;
// s_waitcnt lgkmcnt(0) with the other counters unconstrained.
constexpr int kWaitLgkmcnt0 = 0xC07F;
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
  const int2* wg_units;    // [workgroups]: (first unit, units)
  const int4* units;       // [U][2]: (KV head, first query, q_len, kv_len),
                           //         (q offset, page offset, key tiles, pages)
  int32_t num_kv_heads;
  int32_t causal;
  float scale_log2;        // sm_scale * log2(e)
  uint16_t* out;
  int64_t out_stride;      // elements between output tokens
  float* lse;              // [total_q][Hq] natural log, may be null
};

// K rows of 256 B whose 16-byte chunks are XOR-swizzled by key: chunk c of
// key k sits in slot c ^ (k % 16).
struct alignas(16) KTile { uint8_t b[kKeys * kKRow]; };
// V rows of 256 B, natural [key][dim] layout, 16-byte chunks XOR-swizzled
// as chunk c of key k in slot c ^ 4(k % 4): the transposing reads of four
// consecutive keys then hit distinct banks.
struct alignas(16) VTile { uint8_t b[kKeys * kKRow]; };

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Two floats as a bf16 pair (v_cvt_pk_bf16_f32: round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Eight waves in two teams of four, one workgroup per CU, two waves per SIMD
// (<= 256 VGPRs, no AGPRs): wave w of team 0 and wave w of team 1 share SIMD
// w.  Each team owns 128 query rows and both teams read the same K/V tiles.
// Per 64-key tile a wave has two phases of about equal length: an MFMA phase
// (the 16 MFMAs of O^T += V^T P^T for the previous tile, then the 16 of
// S^T = K Q^T for this tile, LDS operands read ahead, no other work) and a
// VALU phase (the tile's row max, the lazy O rescale, the exponentials, P
// packed to bf16 and summed).  Team 1 runs one phase behind team 0 and every
// phase ends on a workgroup barrier, so on each SIMD one wave's MFMA chain
// runs while the other wave does its softmax: the matrix pipe does not wait
// for the VALU, and the VALU is never starved by the matrix pipe.  The MFMA
// team raises its priority for its phase.
//
// Slots 2j and 2j+1 each end on a workgroup barrier.  M_j: O += P_{j-1}
// V_{j-1} (j >= 1) and S_j = K_j Q (j < ntiles); X_j: softmax of S_j into
// P_j.  Team 0 runs M_j in slot 2j and X_j in slot 2j+1; team 1 runs X_{j-1}
// in slot 2j and M_j in slot 2j+1.  Team 1 also stages: at the start of
// slot 2j each of its waves issues the direct-to-LDS loads of its page
// (w - 4) of K_{j+1} and of V_j (the buffers they overwrite were last read
// in slot 2j-1), from page offsets resolved two tiles earlier, and waits
// for them before the barrier that ends slot 2j+1; page resolution and the
// next page-id fetch come after its softmax, off the MFMA team's path.  The
// softmax is lean: per-key tests only on boundary tiles, the scale folded
// into one FMA per score, the O rescale skipped unless a row max grows by
// more than 2^8, P packed to bf16 with v_cvt_pk_bf16_f32 and summed from the
// packed pairs with v_dot2_f32_bf16, the row max exchanged between the lane
// halves with v_permlane32_swap.
//
// The host plan gives each workgroup a list of units (the list scheduling a
// dispatcher would do, made explicit so that a unit's first loads can be
// issued during the previous unit: its record, its first page ids and, by
// team 1 in the previous unit's slot 2n, its first K tile).

// A work unit's record: (KV head, first query, q_len, kv_len, q offset, page
// offset, key tiles, pages) of one query tile of one request.
struct Unit { int h, tok0, q_len, kv_len, q_off, page_off, ntiles, npages; };

template <int G>
__global__ __launch_bounds__(kThreads, 1) void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int kTokPerWave = kWaveRows / G;
  // One LDS object, so that the K/V tiles sit in its first 64 KB (operand
  // reads then address them with immediate offsets) and the output staging
  // after them: each wave's finished rows on their way out, 32 rows of
  // 256 B padded to kORow (a row's 16 pieces written by one instruction then
  // spread over the banks, and every lane address is a base plus an
  // immediate).
  struct Lds {
    KTile k[2];
    VTile v[2];
    uint8_t ostage[8][kWaveRows * kORow];
  };
  __shared__ Lds lds;
  KTile (&ktiles)[2] = lds.k;
  VTile (&vtiles)[2] = lds.v;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR
  const int team = wave >> 2;
  const int pw_idx = wave & 3;        // the page of a tile this wave stages (team 1)
  const int lane = threadIdx.x & 63;
  const int r = lane & 31;
  const int half = lane >> 5;
  const int g = r % G;
  const int Hq = a.num_kv_heads * G;

  // This workgroup's units, in order: records [first, first + count).
  const int2 span = a.wg_units[blockIdx.x];
  const int u_first = __builtin_amdgcn_readfirstlane(span.x);
  const int u_count = __builtin_amdgcn_readfirstlane(span.y);
  // A unit's record as loaded (VGPRs, no wait) and as used (SGPRs).
  struct RawUnit { int4 x, y; };
  auto fetch_unit = [&](int u) __attribute__((always_inline)) {
    return RawUnit{a.units[2 * u], a.units[2 * u + 1]};
  };
  auto to_unit = [](const RawUnit& t) __attribute__((always_inline)) {
    auto rfl = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    return Unit{rfl(t.x.x), rfl(t.x.y), rfl(t.x.z), rfl(t.x.w),
                rfl(t.y.x), rfl(t.y.y), rfl(t.y.z), rfl(t.y.w)};
  };
  // Q of a unit as the B operand of S^T = K Q^T: k-step ks covers head dims
  // 16ks .. 16ks+15, lane half h the dims 16ks + 8h .. +7.  Rows past the
  // chunk load the chunk's first token (every unit has one): a row's scores,
  // softmax and output involve only its own Q, and such rows are never
  // stored.  Every lane loads, so the loads need no branches around them
  // and the compiler can count them exactly (branches made it wait for all
  // loads in flight, these included, at the unit switch).
  auto load_q = [&](const Unit& U, bf16x8_t (&dst)[kD / 16]) __attribute__((always_inline)) {
    const int t = U.tok0 + wave * kTokPerWave + r / G;
    const uint16_t* qp = a.q + int64_t(U.q_off + (t < U.q_len ? t : 0)) * a.q_stride +
                         int64_t(U.h * G + g) * kD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks)
      dst[ks] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 16 * ks));
  };

  // The current unit and this lane's row in it.
  Unit cu = to_unit(fetch_unit(u_first));
  int tok = 0, limit = -1, hq = 0, n_full = 0;
  bool row_ok = false;
  const int32_t last_index = int32_t(min(a.num_indices - 1, int64_t(INT32_MAX)));
  auto set_unit = [&](const Unit& U) __attribute__((always_inline)) {
    cu = U;
    tok = U.tok0 + wave * kTokPerWave + r / G;
    row_ok = tok < U.q_len;
    // Last key this row may see (inclusive).
    limit = !row_ok ? -1 : a.causal ? min(tok + U.kv_len - U.q_len, U.kv_len - 1) : U.kv_len - 1;
    hq = U.h * G + g;
    // Tiles [0, n_full) are interior for every row of the workgroup (all
    // its rows see keys up to at least its first token's limit).
    const int lim_lo = a.causal ? U.tok0 + U.kv_len - U.q_len : U.kv_len - 1;
    n_full = max(0, min(U.ntiles, (lim_lo + 1) / kKeys));
  };
  set_unit(cu);
  bf16x8_t qb[kD / 16];
  load_q(cu, qb);

  const char* kbase = reinterpret_cast<const char*>(a.k_cache);
  const char* vbase = reinterpret_cast<const char*>(a.v_cache);
  const int64_t tok_bytes = a.token_stride * 2;
  // Direct-to-LDS staging: this wave's load i fetches keys 4i .. 4i+3 of its
  // page, lane L key 4i + L/16, the chunk whose swizzled slot is L%16 (K and
  // V each with their own swizzle), at these offsets from the unit's head
  // slice of the page.
  uint32_t lane_k[4], lane_v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = 4 * i + (lane >> 4);
    lane_k[i] = uint32_t(key * tok_bytes + ((lane & 15) ^ (key & 15)) * 16);
    lane_v[i] = uint32_t(key * tok_bytes + ((lane & 15) ^ (4 * (key & 3))) * 16);
  }
  // Every global_load_lds of this wave has written LDS (vmcnt 0).
  auto wait_dma = []() __attribute__((always_inline)) { __builtin_amdgcn_s_waitcnt(kWaitVmcnt0); };

  // Page ids of a tile as loaded: lane u (u = lane % 4) loads page u at a
  // clamped address, one load per tile, fetched well before the K/V loads
  // need them.  Index arithmetic is 32-bit (the host keeps every page index
  // below 2^31).
  const int32_t num_blocks32 = int32_t(min(a.num_blocks, int64_t(INT32_MAX)));
  struct RawIds { int32_t v; };
  auto fetch_ids = [&](const Unit& U, int tile) __attribute__((always_inline)) {
    return RawIds{a.indices[min(U.page_off + tile * 4 + (lane & 3), last_index)]};
  };
  // Byte offset of this wave's page of a tile, at the unit's head (the host
  // keeps a block stride under 4 GiB), and the tile's present pages: bit u
  // of `ok` says page u is real (inside the request and the cache); the
  // others read block 0 and are masked.  Pages [0, pages_here) of the unit
  // exist in the request and the index array; a present page also needs an
  // id in [0, num_blocks).  The four tests run on lanes 0..3 at once and
  // one ballot collects them.
  const uint32_t blk32 = uint32_t(a.block_stride * 2);
  struct Pages { uint64_t off; int ok; };
  auto resolve = [&](const Unit& U, const RawIds& t, int tile) __attribute__((always_inline)) {
    const int pages_here = min(U.npages, last_index - U.page_off + 1);
    const bool good = (tile * 4 + (lane & 3) < pages_here) & (uint32_t(t.v) < uint32_t(num_blocks32));
    const int ok = int(__builtin_amdgcn_ballot_w64(good) & 0xF);
    const int32_t v = good ? t.v : 0;
    return Pages{uint64_t(uint32_t(__builtin_amdgcn_readlane(v, pw_idx))) * blk32 +
                     uint32_t(U.h * kD * 2), ok};
  };
  // Direct loads from memory into LDS (global_load_lds_dwordx4 and
  // buffer_load_dwordx4 ... lds, one 16-byte chunk per lane, lane L at LDS
  // offset 16L from the wave-uniform address in M0).  They are issued as
  // inline assembly so that the compiler does not make every later LDS read
  // wait for them (it cannot tell the buffer being filled from the one being
  // read); each wave waits for its own (vmcnt 0) before the barrier that
  // publishes the tiles.  No compiler-generated code here uses M0 (M0 is a
  // reserved register hipcc will not take as a clobber;
  // tests/test_prefill_m0.py checks the built assembly for any other use).
  auto lds_addr = [](const void* p) __attribute__((always_inline)) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void_t*)p));
  };
  // A wave-uniform 64-bit value as an SGPR pair (the page offsets are
  // uniform, but the compiler may keep them in VGPRs).
  auto sgpr64 = [](uint64_t v) __attribute__((always_inline)) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return (uint64_t(hi) << 32) | lo;
  };
  // K: one instruction of a wave fills 1 KB of LDS (keys 4i .. 4i+3 of the
  // wave's page); the page's four come from one block address, with M0
  // stepped by 1 KB between them.
  auto dma_k = [&](KTile& buf, const Pages& p) __attribute__((always_inline)) {
    const uint64_t blk = sgpr64(reinterpret_cast<uint64_t>(kbase + p.off));
    asm volatile("s_mov_b32 m0, %0\n\t"
                 "global_load_lds_dwordx4 %1, %5\n\ts_add_u32 m0, m0, 0x400\n\t"
                 "global_load_lds_dwordx4 %2, %5\n\ts_add_u32 m0, m0, 0x400\n\t"
                 "global_load_lds_dwordx4 %3, %5\n\ts_add_u32 m0, m0, 0x400\n\t"
                 "global_load_lds_dwordx4 %4, %5"
                 :: "s"(lds_addr(buf.b + pw_idx * kPage * kKRow)), "v"(lane_k[0]), "v"(lane_k[1]),
                    "v"(lane_k[2]), "v"(lane_k[3]), "s"(blk) : "memory", "scc");
  };
  // V goes into LDS the same way, through a buffer load bounded to the
  // page's valid tokens: lanes past kv_len or in a missing page get zeros
  // (a P of 0 times V bits that happen to be NaN would not be 0).  K needs
  // no such care: a key's score depends on its own K row only, and tiles
  // holding such keys are processed with the per-key tests, which never
  // read its score.
  const int page_bytes = kPage * int(tok_bytes);  // under 2 GiB (host check)
  auto dma_v = [&](VTile& buf, const Pages& p, int kv_len, int tile) __attribute__((always_inline)) {
    const bool real = (p.ok >> pw_idx) & 1;
    int bytes = real ? page_bytes : 0;
    if ((tile + 1) * kKeys > kv_len) {
      const int rem = max(0, min(kPage, kv_len - tile * kKeys - pw_idx * kPage));
      bytes = real ? rem * int(tok_bytes) : 0;
    }
    const uint64_t blk = reinterpret_cast<uint64_t>(vbase + p.off);
    const i32x4_t rsrc = {__builtin_amdgcn_readfirstlane(int(uint32_t(blk))),
                          __builtin_amdgcn_readfirstlane(int(uint32_t(blk >> 32) & 0xFFFF)),
                          __builtin_amdgcn_readfirstlane(bytes), kBufferRsrcWord3};
    asm volatile("s_mov_b32 m0, %0\n\t"
                 "buffer_load_dwordx4 %1, %5, 0 offen lds\n\ts_add_u32 m0, m0, 0x400\n\t"
                 "buffer_load_dwordx4 %2, %5, 0 offen lds\n\ts_add_u32 m0, m0, 0x400\n\t"
                 "buffer_load_dwordx4 %3, %5, 0 offen lds\n\ts_add_u32 m0, m0, 0x400\n\t"
                 "buffer_load_dwordx4 %4, %5, 0 offen lds"
                 :: "s"(lds_addr(buf.b + pw_idx * kPage * kKRow)), "v"(lane_v[0]), "v"(lane_v[1]),
                    "v"(lane_v[2]), "v"(lane_v[3]), "s"(rsrc) : "memory", "scc");
  };

  // V tiles start as zeros: should a bounded load leave the LDS rows of
  // out-of-range lanes untouched, they hold zeros or earlier valid rows,
  // never stale bits from before the kernel.  Each V-staging wave clears the
  // rows its own loads fill (rows 16*(w-4) .. +15 of both buffers) and waits
  // for that before issuing them.
  if (team == 1) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      uint8_t* row = vtiles[c >> 2].b + (pw_idx * kPage + 4 * (c & 3) + (lane >> 4)) * kKRow;
      *reinterpret_cast<uint4*>(row + (lane & 15) * 16) = make_uint4(0, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkmcnt0);
  }

  uint32_t v_rd[4];
  {
    const int e = (lane >> 2) & 3, q = lane & 3, gp = (lane >> 4) & 1, hh = lane >> 5;
#pragma unroll
    for (int db = 0; db < 4; ++db)
      v_rd[db] = (4 * hh + e) * kKRow + ((4 * (db ^ e) + 2 * gp + (q >> 1)) << 4) + ((q & 1) << 3);
  }
  // MFMA operands from LDS.  Score MFMA i (0..15) of a tile: k-step i/2 of
  // key block i%2 (keys 32(i%2) .. +31), A = those keys' dims.  Output MFMA
  // i: key step i/4 (keys 16(i/4) .. +15), head-dim block i%4, A = V^T rows.
  auto k_operand = [&](const KTile& buf, int i) __attribute__((always_inline)) {
    return as_bf16x8(*reinterpret_cast<const uint4*>(
        buf.b + (32 * (i & 1) + r) * kKRow + (((2 * (i >> 1) + half) ^ (r & 15)) << 4)));
  };
  // The V^T operand comes from the [key][dim] tile through two transposing
  // reads (ds_read_b64_tr_b16).  Within a group of 16 lanes, lane j supplies
  // the address of 4 consecutive elements and lane i receives element i%4 of
  // the rows supplied by lanes i/4 + {0,4,8,12}.  So lane j = 4e + q of
  // group g points at key 16st + 4(g/2) + e (+8 for the second read), dims
  // 32db + 16(g%2) + 4q .. +3, and lane i of the group receives dim
  // 32db + 16(g%2) + i for the four keys -- the rows and key order of the
  // P^T operand.  v_rd[db]: this lane's address for k-step 0.
  auto v_operand = [&](const VTile& buf, int i) __attribute__((always_inline)) {
    const uint8_t* p = buf.b + v_rd[i & 3] + (i >> 2) * 16 * kKRow;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + 8 * kKRow));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16_t o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  f32x16_t s[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
  uint32_t pw[2][8];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 8; ++e) pw[kb][e] = 0u;
  // m_run: the row's running max (base 2, scaled); l_half: the running sum
  // of p over this lane's half of every tile's keys (lane l^32 holds the
  // other half), both under the same m_run.
  float m_run = kNegBig, l_half = 0.f;
  const uint32_t ones = 0x3F803F80u;  // bf16 pair (1, 1)

  // Accumulator entry e of key block kb holds key 32kb + 8(e/4) + 4half + e%4
  // of the tile, which lies in page 2kb + e/8 of the tile.  Interior tiles
  // (every key visible to every row of the workgroup, all pages present)
  // skip the per-key tests.  rel = the key offset (within the lane's half of
  // the tile) the row may still see.
  auto visible = [&](int rel, int ok, int kb, int e) __attribute__((always_inline)) {
    return (32 * kb + 8 * (e >> 2) + (e & 3)) <= rel && ((ok >> (2 * kb + (e >> 3))) & 1);
  };
  // M_j: O += P_{j-1} V_{j-1} (do_o), then S_j = K_j Q (do_s), each MFMA's
  // LDS operand read four MFMAs ahead.
  auto mfma_phase = [&](int j, auto do_o_c, auto do_s_c) __attribute__((always_inline)) {
    if constexpr (decltype(do_o_c)::value) {
      const VTile& vb = vtiles[(j - 1) & 1];
      bf16x8_t vop[16];
#pragma unroll
      for (int i = 0; i < 3; ++i) vop[i] = v_operand(vb, i);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i + 3 < 16) vop[i + 3] = v_operand(vb, i + 3);
        const int st = i >> 2;
        const uint32_t* pp = &pw[st >> 1][4 * (st & 1)];
        const bf16x8_t pb = as_bf16x8(make_uint4(pp[0], pp[1], pp[2], pp[3]));
        o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop[i], pb, o[i & 3], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (decltype(do_s_c)::value) {
      const KTile& kb = ktiles[j & 1];
      const f32x16_t zero = {};
      bf16x8_t kop[16];
#pragma unroll
      for (int i = 0; i < 3; ++i) kop[i] = k_operand(kb, i);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i + 3 < 16) kop[i + 3] = k_operand(kb, i + 3);
        s[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[i], qb[i >> 1],
                                                           i < 2 ? zero : s[i & 1], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // X_j: on a tile that needs the per-key tests (a boundary tile or a
  // missing page) the scores of keys the row may not see become -inf, in
  // place (the exponentials then need no tests: exp2(-inf) = 0, the scale
  // being positive and finite); then the row max of S_j is folded into m_run
  // with the lazy rescale of O and l, and P_j = exp2(S scale - m_run) is
  // packed to bf16 in S^T accumulator order and summed into l_half.  The
  // masking is a block of its own that only rewrites S, so O has one path
  // through the phase.
  auto valu_phase = [&](int j, int ok) __attribute__((always_inline)) {
    if (!(j < n_full && ok == 0xF)) {
      const int rel = limit - j * kKeys - 4 * half;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[kb][e] = visible(rel, ok, kb, e) ? s[kb][e] : -INFINITY;
    }
    float mx = kNegBig;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kb][e]);
    // Fold the tile's row max (this lane's 32 keys and lane l^32's; the raw
    // scores, as the scale is positive) into the running max.  A row's
    // running max only moves when its max grew by more than kRescaleLog2
    // (base-2 units); otherwise the stale max stays, p <= 2^8, and the
    // rescale of O and l is skipped.  Each row decides for itself, so a
    // row's result does not depend on which other rows share its wave.
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                     false, false);
    mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    const float cand = fmaxf(m_run, mx * a.scale_log2);
    const bool grow = cand > m_run + kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float alpha = grow ? fast_exp2(m_run - cand) : 1.f;
      m_run = grow ? cand : m_run;
      l_half *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
    float sum0 = 0.f, sum1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kb = i >> 3, e = 2 * (i & 7);
      const float p0 = fast_exp2(fmaf(s[kb][e], a.scale_log2, -m_run));
      const float p1 = fast_exp2(fmaf(s[kb][e + 1], a.scale_log2, -m_run));
      pw[kb][e >> 1] = pack_bf16(p0, p1);
      if (i & 1) sum1 = dot2_bf16(pw[kb][e >> 1], ones, sum1);
      else sum0 = dot2_bf16(pw[kb][e >> 1], ones, sum0);
      if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    l_half += sum0 + sum1;
  };

  // The unit's output rows: O / l in bf16 and, when asked, the natural-log
  // log-sum-exp; then the running state starts over for the next unit.  The
  // rows go out through this wave's LDS staging: each lane holds 8-byte
  // pieces of one row, which as stores would touch 32 rows per instruction;
  // read back, lane L of store t holds 16 bytes of row 4t + L/16, so a store
  // writes four whole rows (one token's four heads at G = 4: 1 KB in a run).
  // The stores are non-temporal: the output is not read again here, and
  // leaving it out of the caches keeps the K/V tiles the other query tiles
  // of a request re-read there.
  auto finish_unit = [&]() __attribute__((always_inline)) {
    const float l_run = l_half + __shfl_xor(l_half, 32);
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    uint8_t* stg = lds.ostage[wave];
    // O^T column r = this row; entry (db, 4i+j) = head dim 32db + 8i + 4half + j,
    // so (db, i) is the row's 16-byte chunk 4db + i and half its 8-byte half.
    uint8_t* wr = stg + r * kORow + 8 * half;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint2*>(wr + 16 * (4 * db + i)) =
            make_uint2(pack_bf16(o[db][4 * i] * inv, o[db][4 * i + 1] * inv),
                       pack_bf16(o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv));
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Row 4t + q (q = L/16 < 4) is token (4t + q) / G of the wave, head
    // (4t + q) % G: for G <= 4 that is token t (4/G) + q/G, head q % G; for
    // G >= 4 token 4t/G, head 4t % G + q.  So the lane's part of the address
    // is set once and the store's part is uniform.
    const int c = lane & 15;
    const int q = lane >> 4;
    const int wave_tok = cu.tok0 + wave * kTokPerWave;
    const int toks_left = cu.q_len - wave_tok;
    const int lane_tok = G <= 4 ? q / G : 0;
    const int lane_head = G <= 4 ? q % G : q;
    uint16_t* obase = a.out + int64_t(cu.q_off + wave_tok + lane_tok) * a.out_stride +
                      int64_t(cu.h * G + lane_head) * kD + 8 * c;
    const uint8_t* rd = stg + q * kORow + 16 * c;
    // Four read-backs in flight, then their four stores (one at a time, each
    // store waited for its own read).
#pragma unroll
    for (int t0 = 0; t0 < kWaveRows / 4; t0 += 4) {
      uint4 v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = *reinterpret_cast<const uint4*>(rd + 4 * (t0 + i) * kORow);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + i;
        const int t_tok = G <= 4 ? t * (4 / G) : 4 * t / G;
        const int t_head = G <= 4 ? 0 : 4 * t % G;
        if (t_tok + lane_tok < toks_left)
          store_stream(obase + int64_t(t_tok) * a.out_stride + t_head * kD, v[i]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (row_ok && a.lse && half == 0)
      a.lse[int64_t(cu.q_off + tok) * Hq + hq] =
          l_run > 0.f ? (m_run + fast_log2(l_run)) * kLn2 : -INFINITY;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
    m_run = kNegBig;
    l_half = 0.f;
  };

  // Per unit with n key tiles, slots 2j and 2j+1 (each ends on a workgroup
  // barrier): team 0 runs M_j then X_j, team 1 runs X_{j-1} then M_j, for j
  // = 0 .. n (M_0 without O, M_n without S).  Each team has its own copy of
  // the code (the team is a compile-time constant in `run`), with the first
  // and last tiles peeled, so the loop body is straight-line code in which
  // O, S and P keep their registers; the teams only have to meet the same
  // barriers, not the same instructions.  While a unit runs, the next one's
  // record and first page ids are fetched, its Q is loaded once this unit's
  // last S_j is done, and team 1 stages its first K tile in slot 2n.  A
  // unit whose first K tile was not staged that way (the workgroup's first,
  // or one after a unit without key tiles) starts with a staging step of its
  // own.
  using yes = std::true_type;
  using no = std::false_type;
  auto run = [&](auto team_c) __attribute__((always_inline)) {
    constexpr int kTeam = decltype(team_c)::value;
    auto mfma = [&](int j, auto do_o_c, auto do_s_c) __attribute__((always_inline)) {
      __builtin_amdgcn_s_setprio(1);
      mfma_phase(j, do_o_c, do_s_c);
      __builtin_amdgcn_s_setprio(0);
    };
    Unit nu = u_count > 1 ? to_unit(fetch_unit(u_first + 1)) : cu;  // the next unit
    RawUnit nnu{};                                                   // the one after
    RawIds c0 = fetch_ids(cu, 0), c1 = fetch_ids(cu, 1);     // current unit's tiles 0, 1
    RawIds n0{0}, n1{0}, n2{0};                             // next unit's tiles 0..2
    bool staged = false;      // the current unit's K_0 is in ktiles[0] (team 1 state too)
    Pages pv{0, 0}, pk{0, 0};  // team 1: pages of tiles j and j+1
    RawIds raw{0};             // team 1: ids of tile j+2; team 0: of tile j+1
    // After unit k's own first loads: the next unit's page ids and the
    // record of the unit after it.
    auto prefetch_next = [&](int k) __attribute__((always_inline)) {
      if (k + 1 < u_count) {
        n0 = fetch_ids(nu, 0);
        n1 = fetch_ids(nu, 1);
        n2 = fetch_ids(nu, 2);
        if (k + 2 < u_count) nnu = fetch_unit(u_first + k + 2);
      }
    };
    for (int k = 0; k < u_count; ++k) {
      const bool has_next = k + 1 < u_count;
      const int n = cu.ntiles;
      if (n > 0) {
        if (kTeam == 0) {
          // Team 0 stages nothing; it only needs each tile's present pages
          // for its VALU phase, resolved one tile ahead after that phase.
          if (!staged) __syncthreads();
          mfma(0, no{}, yes{});
          __syncthreads();
          int ok_cur = resolve(cu, c0, 0).ok;  // tile j's, from slot 2j+1 on
          valu_phase(0, ok_cur);
          ok_cur = resolve(cu, c1, 1).ok;
          raw = fetch_ids(cu, 2);
          prefetch_next(k);
          __syncthreads();
          for (int j = 1; j < n; ++j) {
            mfma(j, yes{}, yes{});
            __syncthreads();
            valu_phase(j, ok_cur);
            ok_cur = resolve(cu, raw, j + 1).ok;
            raw = fetch_ids(cu, j + 2);
            __syncthreads();
          }
          // Q is not read again in this unit: the next unit's goes into its
          // registers two slots before that unit's first MFMA phase.
          if (has_next) load_q(nu, qb);
          mfma(n, yes{}, no{});
          __syncthreads();
          finish_unit();
          __syncthreads();
        } else {
          // Team 1 stages K_{j+1} and V_j at the start of slot 2j, from
          // pages resolved two tiles ahead, and waits for them at the end of
          // slot 2j+1.
          int ok_prev = 0;                     // tile j-1's present pages
          // After slot 2j's loads are issued: resolve tile j+2, fetch tile
          // j+3's page ids and shift the window.
          auto advance = [&](int j) __attribute__((always_inline)) {
            const Pages pn = resolve(cu, raw, j + 2);
            raw = fetch_ids(cu, j + 3);
            ok_prev = pv.ok;
            pv = pk;
            pk = pn;
          };
          if (!staged) {
            raw = fetch_ids(cu, 2);
            pv = resolve(cu, c0, 0);
            pk = resolve(cu, c1, 1);
            dma_k(ktiles[0], pv);
            wait_dma();
            __syncthreads();
          }
          if (1 < n) dma_k(ktiles[1], pk);
          dma_v(vtiles[0], pv, cu.kv_len, 0);
          advance(0);
          prefetch_next(k);
          __syncthreads();
          mfma(0, no{}, yes{});
          wait_dma();
          __syncthreads();
          for (int j = 1; j < n; ++j) {
            if (j + 1 < n) dma_k(ktiles[(j + 1) & 1], pk);
            dma_v(vtiles[j & 1], pv, cu.kv_len, j);
            valu_phase(j - 1, ok_prev);
            advance(j);
            __syncthreads();
            mfma(j, yes{}, yes{});
            wait_dma();
            __syncthreads();
          }
          valu_phase(n - 1, ok_prev);
          // Q is not read again in this unit (its last S_j was in slot
          // 2n-1): the next unit's goes into its registers, waited for with
          // this slot's loads.  The next unit's first K tile goes into
          // ktiles[0], last read in slot 2n-1 or earlier.
          if (has_next) load_q(nu, qb);
          if (has_next && nu.ntiles > 0) {
            pv = resolve(nu, n0, 0);
            pk = resolve(nu, n1, 1);
            raw = n2;
            dma_k(ktiles[0], pv);
          }
          __syncthreads();
          mfma(n, yes{}, no{});
          wait_dma();
          __syncthreads();
          finish_unit();
        }
      } else {
        prefetch_next(k);
        if (has_next) load_q(nu, qb);
        finish_unit();
      }
      if (has_next) {
        staged = n > 0 && nu.ntiles > 0;
        set_unit(nu);
        if (k + 2 < u_count) nu = to_unit(nnu);
        c0 = n0;
        c1 = n1;
      }
    }
  };
  if (team == 0) run(std::integral_constant<int, 0>{});
  else run(std::integral_constant<int, 1>{});
}

template <int G>
void launch(const PrefillArgs& a, int workgroups, hipStream_t s) {
  prefill_mfma_kernel<G><<<dim3(unsigned(workgroups)), kThreads, 0, s>>>(a);
}

// Persistent workgroups: at most one per CU of an MI355X (256), each running
// a list of units; the plan image is the workgroups' (first unit, units)
// table, padded to 4 int32, then the unit records.
constexpr int64_t kMaxWorkgroups = 256;
int64_t plan_workgroups(int64_t items, int hkv) { return std::min(kMaxWorkgroups, items * hkv); }
int64_t plan_table_ints(int64_t workgroups) { return (2 * workgroups + 3) / 4 * 4; }
int64_t plan_ints_for(int64_t items, int hkv) {
  return plan_table_ints(plan_workgroups(items, hkv)) + items * hkv * kItemInts;
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
  KVC_REQUIRE(n * num_kv_heads < (int64_t(1) << 30), KVC_ERR_INVALID_ARG,
              "too many (query tile, KV head) units");
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
  sched->plan_ints = plan_ints_for(n, num_kv_heads);
  KVC_REQUIRE(plan_host && plan_capacity >= sched->plan_ints, KVC_ERR_WORKSPACE,
              "plan buffer too small: need " + std::to_string(sched->plan_ints) + " int32");
  // Longest items first: the causal tail of short tiles fills the gaps.
  std::vector<int64_t> order(n);
  for (int64_t i = 0; i < n; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int64_t x, int64_t y) {
    return rec[x * kItemInts + 6] > rec[y * kItemInts + 6];
  });
  // Units (item, KV head) in the order a grid of (items, heads) workgroups
  // would be dispatched: head-major, items longest first.  The hardware
  // hands workgroup w to XCD w % 8 and each XCD's next workgroup to its
  // first free CU; the plan replays that list scheduling with each unit's
  // cost taken as its key tiles + 2, assigning unit d to a workgroup of XCD
  // d % 8 (workgroup b runs on XCD b % 8), so the units of one request and
  // head still run side by side on one XCD and share its L2.
  const int64_t units = n * num_kv_heads;
  const int64_t W = plan_workgroups(n, num_kv_heads);
  const int groups = (W % 8 == 0) ? 8 : 1;
  std::vector<std::vector<int64_t>> lists(W);
  {
    typedef std::pair<int64_t, int64_t> Slot;  // (load, workgroup)
    std::vector<std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>>> free_at(groups);
    for (int64_t b = 0; b < W; ++b) free_at[b % groups].push(Slot(0, b));
    for (int64_t d = 0; d < units; ++d) {
      auto& q = free_at[d % groups];
      const Slot sl = q.top();
      q.pop();
      lists[sl.second].push_back(d);
      const int64_t item = order[d % n];
      q.push(Slot(sl.first + rec[item * kItemInts + 6] + 2, sl.second));
    }
  }
  const int64_t table = plan_table_ints(W);
  std::fill_n(plan_host, table, 0);
  int64_t next = 0;
  for (int64_t b = 0; b < W; ++b) {
    plan_host[2 * b] = int32_t(next);
    plan_host[2 * b + 1] = int32_t(lists[b].size());
    for (const int64_t d : lists[b]) {
      int32_t* dst = plan_host + table + next * kItemInts;
      std::copy_n(rec.data() + order[d % n] * kItemInts, kItemInts, dst);
      dst[0] = int32_t(d / n);  // the KV head
      ++next;
    }
  }
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
                  sched->tile_tokens == kTileRows / (Hq / Hkv) && sched->num_items >= 0 &&
                  sched->plan_ints == plan_ints_for(sched->num_items, Hkv),
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
  KVC_REQUIRE(cache_block_stride * 2 < (int64_t(1) << 32), KVC_ERR_INVALID_ARG,
              "cache blocks 4 GiB or more apart");
  KVC_REQUIRE(q_token_stride >= int64_t(Hq) * kD && out_token_stride >= int64_t(Hq) * kD,
              KVC_ERR_INVALID_ARG, "q/out token stride smaller than Hq*head_dim");
  KVC_REQUIRE(sm_scale > 0.f && std::isfinite(sm_scale), KVC_ERR_INVALID_ARG,
              "sm_scale must be positive and finite");
  KVC_REQUIRE(aligned(q, 16) && aligned(key_cache, 16) && aligned(value_cache, 16) &&
                  aligned(out, 16) && aligned(plan, 16) && q_token_stride % 8 == 0 &&
                  out_token_stride % 8 == 0 && cache_block_stride % 8 == 0 &&
                  cache_token_stride % 8 == 0,
              KVC_ERR_ALIGNMENT, "q/out/cache/plan must be 16-byte aligned with matching "
                                 "strides");
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
  const int64_t workgroups = plan_workgroups(sched->num_items, Hkv);
  a.wg_units = reinterpret_cast<const int2*>(plan);
  a.units = reinterpret_cast<const int4*>(plan + plan_table_ints(workgroups));
  a.num_kv_heads = Hkv;
  a.causal = sched->causal;
  a.scale_log2 = sm_scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.out_stride = out_token_stride;
  a.lse = lse;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (Hq / Hkv) {
    case 1: launch<1>(a, int(workgroups), s); break;
    case 2: launch<2>(a, int(workgroups), s); break;
    case 4: launch<4>(a, int(workgroups), s); break;
    case 8: launch<8>(a, int(workgroups), s); break;
    default: KVC_REQUIRE(false, KVC_ERR_UNSUPPORTED, "group must be 1, 2, 4 or 8");
  }
  KVC_LAUNCH_CHECK();
  return ok();
}
