// vLLM's "x-packed" paged KV layout, the second on-device KV format of the
// reference (its dense sandbox, src/dense/include/paged_transformer.py:85-92):
//   key_cache   [num_blocks, H, D/x, block_size, x]   x = 16 bytes / element
//   value_cache [num_blocks, H, D, block_size]
// with vLLM's reshape_and_cache writing it (:290-294) and
// paged_attention_v1/v2 reading it (:325-332; src/dense/scratch_examples/
// vllm_paged_attn.py:274-288).  fp16 and bf16 (2-byte elements, x = 8),
// head_size 128, block_size 16.
//
// In this layout one (block, head) is a contiguous 4 KB of K and 4 KB of V,
// so decode streams straight into registers, no LDS staging:
//   q.k : lane (token t = l%16, chunk group cg = l/16) loads the 16-byte
//         chunks 4cg..4cg+3 of token t (dims 32cg..32cg+31), 16 dot2 per query
//         head, then two xor-shuffles sum the 4 chunk groups;
//   p.v : lane l loads 16 B at 16l + 1024j (dim l/2 + 32j, tokens 8(l%2) ..
//         +7; every load one contiguous KB); p is rounded to the cache dtype
//         in (t, t+1) pairs -- as vLLM's kernel does before its value dot --
//         broadcast with v_readlane and folded with 4 dot2 per dim; lanes l
//         and l^1 add their token halves at the end.
// Block ids are loaded 64 pages at a time, one per lane, and broadcast.
// A workgroup (4 waves) owns one KV head x one 512-token partition (v2) or the
// whole sequence (v1); wave w takes pages w, w+4, ...; the waves' softmax
// states are merged through LDS.  v2 leaves vLLM's per-partition max logit,
// exp-sum and normalised partial output, and a reduce kernel combines them.
#include "kvc_common.h"

#include <algorithm>
#include <cmath>

namespace kvc {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kV2Waves = 4;  // waves per v2 workgroup (1, 2 and 4 measured alike)
constexpr int kBlock = 16;    // tokens per block
constexpr int kD = 128;       // head size
constexpr int kX = 8;         // elements per 16-byte chunk
constexpr int kPart = 512;    // tokens per v2 partition (vLLM's)
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;

template <bool kBf16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (kBf16)
    return dot2_bf16(a, b, c);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                  __builtin_bit_cast(half2_t, b), c, false);
}

// float -> element bits, round to nearest even.
template <bool kBf16>
__device__ __forceinline__ uint32_t to_elem(float f) {
  if constexpr (kBf16)
    return f32_to_bf16(f);
  else
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <bool kBf16>
__device__ __forceinline__ float from_elem(uint32_t bits) {
  if constexpr (kBf16)
    return __uint_as_float(bits << 16);
  else
    return static_cast<float>(__builtin_bit_cast(_Float16, uint16_t(bits)));
}

// ------------------------------------------------------------------ append
struct XAppendArgs {
  const uint16_t* key;
  const uint16_t* value;
  uint16_t* key_cache;
  uint16_t* value_cache;
  const int64_t* slots;
  int64_t key_stride;      // elements between source tokens
  int64_t value_stride;
  int64_t block_stride;    // elements between cache blocks (K and V)
  int64_t head_stride;     // elements between heads of a block (K and V)
  int64_t num_slots;
  int64_t num_tokens;
  int32_t num_heads;
  int32_t* oob_count;
};

// Workgroup = 16 consecutive tokens x one head; thread (t, c) = (j/16, j%16)
// reads 16-byte chunk c of token t's K and V rows (coalesced: 16 threads per
// 256-byte row).  K chunk c of the token lands on key_cache[blk][h][c][off]
// whole.  V goes to value_cache[blk][h][d][off], one element per dim; when
// the 16 tokens fill one block in order (prefill), the workgroup transposes V
// through LDS and writes each dim's 16 tokens as whole 16-byte runs,
// otherwise (scattered decode slots) it stores the 8 elements one by one.
__global__ __launch_bounds__(kThreads) void xpacked_append_kernel(XAppendArgs a) {
  __shared__ __align__(16) uint16_t s_v[kBlock][kD + 8];
  // Workgroup w = (16-token group w / H, head w % H): the heads of one token
  // group run back to back, so neighbouring workgroups read neighbouring
  // 256-byte slices of the same source rows and write neighbouring 4 KB
  // (block, head) runs of the cache (4.7 -> 5.1 TB/s on a 16K-token prefill,
  // together with the early source loads below).
  const int h = int(blockIdx.x % unsigned(a.num_heads));
  const int64_t grp = blockIdx.x / unsigned(a.num_heads);
  const int t = threadIdx.x >> 4, c = threadIdx.x & 15;
  const int64_t i0 = grp * kBlock;
  const int64_t i = i0 + t;
  const bool live = i < a.num_tokens;
  // The source rows are read together with the slots (their addresses do
  // not depend on them), with the non-temporal hint: they are read once
  // (5.02 -> 5.15 TB/s on a 16K-token prefill).
  uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
  if (live) {
    kv = load_stream(a.key + i * a.key_stride + int64_t(h) * kD + c * kX);
    vv = load_stream(a.value + i * a.value_stride + int64_t(h) * kD + c * kX);
  }
  const int64_t slot = live ? a.slots[i] : -1;
  const int64_t slot0 = a.slots[i0];
  const bool in_range = slot >= 0 && slot < a.num_slots;
  const bool whole = __syncthreads_and(in_range && slot0 % kBlock == 0 && slot == slot0 + t);
  if (slot >= a.num_slots && h == 0 && c == 0 && a.oob_count) atomicAdd(a.oob_count, 1);
  const int64_t blk = slot / kBlock;
  const int off = int(slot % kBlock);
  const int64_t base = blk * a.block_stride + int64_t(h) * a.head_stride;
  if (in_range)
    store_stream(a.key_cache + base + (int64_t(c) * kBlock + off) * kX, kv);
  if (whole) {
    *reinterpret_cast<uint4*>(&s_v[t][c * kX]) = vv;
    __syncthreads();
    // thread j: dim j/2, tokens 8(j%2) .. +7 of the block
    const int d = threadIdx.x >> 1, tb = 8 * (threadIdx.x & 1);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = uint32_t(s_v[tb + 2 * e][d]) | (uint32_t(s_v[tb + 2 * e + 1][d]) << 16);
    const int64_t base0 = (slot0 / kBlock) * a.block_stride + int64_t(h) * a.head_stride;
    store_stream(a.value_cache + base0 + int64_t(d) * kBlock + tb, make_uint4(w[0], w[1], w[2], w[3]));
  } else if (in_range) {
    uint16_t* vdst = a.value_cache + base + int64_t(c) * kX * kBlock + off;
    const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int e = 0; e < kX; ++e)
      vdst[e * kBlock] = uint16_t(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu);
  }
}

// ------------------------------------------------------------------ decode
struct XDecodeArgs {
  const uint16_t* q;
  int64_t q_stride;        // elements between sequences
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t block_stride;
  int64_t head_stride;
  int64_t num_blocks;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t bt_cols;         // entries per block-table row
  const int32_t* seq_lens;
  int32_t num_kv_heads;
  int32_t max_parts;       // partitions per (sequence, head) in the v2 scratch
  int32_t grid_parts;      // partitions launched (ceil(max_seq_len / 512))
  float scale_log2;
  uint16_t* out;           // [seqs][H][D]
  float* exp_sums;         // [seqs][H][max_parts]
  float* max_logits;
  uint16_t* tmp_out;       // [seqs][H][max_parts][D]
};

template <int G, bool kBf16, bool kV1, int kW>
__global__ __launch_bounds__(64 * kW) void xpacked_decode_kernel(XDecodeArgs a) {
  // Grid (KV head, sequence, partition): consecutive workgroups -- which the
  // dispatcher deals to different XCDs -- are heads of one (sequence,
  // partition), i.e. equal work.  (Partition-fastest order put every
  // sequence's partition p on XCD p % 8 and left the XCDs of the late,
  // mostly absent, partitions idle: 4.7 -> 6+ TB/s on a 64-sequence batch.)
  const int h = blockIdx.x, b = blockIdx.y, part = blockIdx.z;
  const int seq_len = max(a.seq_lens[b], 0);
  const int t_begin = kV1 ? 0 : part * kPart;
  const int t_end = kV1 ? seq_len : min(seq_len, t_begin + kPart);
  if (!kV1 && t_begin >= seq_len) return;  // the reduce never reads it
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = lane & 15, cg = lane >> 4;
  const int Hq = a.num_kv_heads * G;

  uint32_t qw[G][16];  // dims 32cg .. 32cg+31 of each query head, as pairs
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint16_t* qp = a.q + int64_t(b) * a.q_stride + int64_t(h * G + g) * kD + 32 * cg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(qp)[i];
      qw[g][4 * i] = v.x; qw[g][4 * i + 1] = v.y; qw[g][4 * i + 2] = v.z; qw[g][4 * i + 3] = v.w;
    }
  }
  float m[G], l[G], acc[G][4];  // acc[g][j]: dim lane/2 + 32j, half of the tokens
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[g][j] = 0.f;
  }

  const int p_begin = t_begin / kBlock, p_end = (t_end + kBlock - 1) / kBlock;
  const int32_t* bt = a.block_tables + int64_t(b) * a.bt_stride;
  // This wave's pages: p_begin + wave + 4j, j < n_pages.  Their block ids
  // are loaded 64 at a time, one per lane, and broadcast with v_readlane.
  const int first = p_begin + wave;
  const int n_pages = p_end > first ? (p_end - first + kW - 1) / kW : 0;
  int32_t id_reg = -1;
  auto id_at = [&](int jj) __attribute__((always_inline)) {
    if ((jj & 63) == 0) {
      const int p = first + kW * (jj + lane);
      const int32_t id = (jj + lane < n_pages && p < a.bt_cols) ? bt[p] : -1;
      id_reg = (id >= 0 && id < a.num_blocks) ? id : -1;
    }
    return __builtin_amdgcn_readlane(id_reg, jj & 63);
  };
  // V of a (block, head) is [D][16 tokens]; lane l loads bytes 16l + 1024j,
  // i.e. dim l/2 + 32j, tokens 8(l%2) .. +7 -- one contiguous KB per load.
  struct Regs { uint4 k[4], v[4]; };
  const int vt0 = 8 * (lane & 1);
  auto load = [&](Regs& r, int32_t id) __attribute__((always_inline)) {
    const int64_t base = int64_t(id < 0 ? 0 : id) * a.block_stride + int64_t(h) * a.head_stride;
    const uint16_t* kb = a.k_cache + base + (int64_t(4 * cg) * kBlock + t) * kX;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.k[i] = load_stream(kb + i * kBlock * kX);
    const uint16_t* vb = a.v_cache + base + lane * kX;
#pragma unroll
    for (int j = 0; j < 4; ++j) r.v[j] = load_stream(vb + j * 64 * kX);
  };
  auto consume = [&](Regs& r, int p, int32_t id) __attribute__((always_inline)) {
    const int valid = id < 0 ? 0 : min(kBlock, t_end - p * kBlock);
    uint32_t* vw = reinterpret_cast<uint32_t*>(r.v);  // [dim j][token pair k]
    if (valid < kBlock) {
      // tokens past the end: zero their V halves (they may hold NaN bits)
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        const int tok = vt0 + 2 * (w & 3);
        vw[w] &= (tok < valid ? 0xffffu : 0u) | (tok + 1 < valid ? 0xffff0000u : 0u);
      }
    }
    const bool live = t < valid;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d = dot2<kBf16>(qw[g][4 * i + 0], r.k[i].x, d);
        d = dot2<kBf16>(qw[g][4 * i + 1], r.k[i].y, d);
        d = dot2<kBf16>(qw[g][4 * i + 2], r.k[i].z, d);
        d = dot2<kBf16>(qw[g][4 * i + 3], r.k[i].w, d);
      }
      d += __shfl_xor(d, 16);
      d += __shfl_xor(d, 32);
      const float s = live ? d * a.scale_log2 : kNegBig;
      const float m_new = fmaxf(m[g], row16_max(s));
      const float pr = live ? fast_exp2(s - m_new) : 0.f;
      const float alpha = fast_exp2(m[g] - m_new);
      l[g] = fmaf(l[g], alpha, row16_sum(pr));
      m[g] = m_new;
      // (p[t], p[t+1]) as one element pair in even lanes, broadcast; this
      // lane needs the pairs of tokens vt0 .. vt0+7.
      const float nxt = __shfl_down(pr, 1, 16);
      const uint32_t pair = to_elem<kBf16>(pr) | (to_elem<kBf16>(nxt) << 16);
      uint32_t pw[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo = __builtin_amdgcn_readlane(pair, 2 * k);
        const uint32_t hi = __builtin_amdgcn_readlane(pair, 8 + 2 * k);
        pw[k] = vt0 ? hi : lo;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float o = acc[g][j] * alpha;
#pragma unroll
        for (int k = 0; k < 4; ++k) o = dot2<kBf16>(pw[k], vw[4 * j + k], o);
        acc[g][j] = o;
      }
    }
  };

  // Two register stages: the wave's next page is in flight while one is consumed.
  Regs ra, rb;
  int32_t ida = -1, idb = -1;
  if (n_pages > 0) { ida = id_at(0); load(ra, ida); }
  for (int j = 0; j < n_pages; j += 2) {
    if (j + 1 < n_pages) { idb = id_at(j + 1); load(rb, idb); }
    consume(ra, first + kW * j, ida);
    if (j + 1 >= n_pages) break;
    if (j + 2 < n_pages) { ida = id_at(j + 2); load(ra, ida); }
    consume(rb, first + kW * (j + 1), idb);
  }
  // the two token halves of each dim live in lanes l and l^1
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[g][j] += __shfl_xor(acc[g][j], 1);

  // Merge the 4 waves' states.
  __shared__ float s_m[kW][G], s_l[kW][G];
  __shared__ float s_acc[kW][G][kD];
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < G; ++g) { s_m[wave][g] = m[g]; s_l[wave][g] = l[g]; }
  if ((lane & 1) == 0)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_acc[wave][g][(lane >> 1) + 32 * j] = acc[g][j];
  __syncthreads();
  // Thread j < G*D: head g = j / D, dim d = j % D.
  for (int j = threadIdx.x; j < G * kD; j += 64 * kW) {
    const int g = j / kD, d = j % kD;
    float mx = kNegBig;
#pragma unroll
    for (int w = 0; w < kW; ++w) mx = fmaxf(mx, s_m[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const float sc = fast_exp2(s_m[w][g] - mx);
      L = fmaf(s_l[w][g], sc, L);
      O = fmaf(s_acc[w][g][d], sc, O);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int hq = h * G + g;
    if constexpr (kV1) {
      a.out[(int64_t(b) * Hq + hq) * kD + d] = uint16_t(to_elem<kBf16>(O * inv));
    } else {
      const int64_t row = (int64_t(b) * Hq + hq) * a.max_parts + part;
      a.tmp_out[row * kD + d] = uint16_t(to_elem<kBf16>(O * inv));
      if (d == 0) {
        a.exp_sums[row] = L;
        a.max_logits[row] = L > 0.f ? mx * kLn2 : -INFINITY;
      }
    }
  }
}

// v2 reduce (vLLM's rule): M = max_p max_logits[p], w_p = exp_sums[p] *
// exp(max_logits[p] - M), out = sum_p w_p tmp_out[p] / sum_p w_p.  One
// partition: out = tmp_out[0].  Workgroup = (query head, sequence), 256
// threads: the partitions' weights are computed in chunks of 256 into LDS,
// then thread (dim d, half r) sums every other partition of the chunk with
// four loads in flight, and the halves are added through LDS.
constexpr int kRedThreads = 256;
template <bool kBf16>
__global__ __launch_bounds__(kRedThreads) void xpacked_reduce_kernel(XDecodeArgs a) {
  __shared__ float s_w[kRedThreads];
  __shared__ float s_part[kRedThreads / 64];
  __shared__ float s_o[2][kD];
  const int hq = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int Hq = gridDim.x;
  const int seq_len = max(a.seq_lens[b], 0);
  const int parts = min((seq_len + kPart - 1) / kPart, a.grid_parts);
  const int64_t row = (int64_t(b) * Hq + hq) * a.max_parts;
  uint16_t* dst = a.out + (int64_t(b) * Hq + hq) * kD;
  if (parts <= 1) {
    if (tid < kD) dst[tid] = parts == 1 ? a.tmp_out[row * kD + tid] : uint16_t(0);
    return;
  }
  // global max logit
  float mx = -INFINITY;
  for (int p = tid; p < parts; p += kRedThreads) mx = fmaxf(mx, a.max_logits[row + p]);
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((tid & 63) == 0) s_part[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_part[0], s_part[1]), fmaxf(s_part[2], s_part[3]));
  const int d = tid & (kD - 1), r = tid >> 7;  // two halves of 128 threads
  float O[2] = {0.f, 0.f}, S = 0.f;
  for (int c0 = 0; c0 < parts; c0 += kRedThreads) {
    __syncthreads();  // s_w of the previous chunk is consumed
    {
      const int p = c0 + tid;
      float w = 0.f;
      if (p < parts) {
        const float lg = a.max_logits[row + p];
        w = lg == -INFINITY ? 0.f : a.exp_sums[row + p] * fast_exp2((lg - mx) * kLog2e);
      }
      s_w[tid] = w;
      S += w;
    }
    __syncthreads();
    const int n = min(kRedThreads, parts - c0);
    const uint16_t* src = a.tmp_out + (row + c0) * kD + d;
    int p = r;
    for (; p + 6 < n; p += 8) {  // four partitions per half in flight
      const float v0 = from_elem<kBf16>(src[int64_t(p) * kD]);
      const float v1 = from_elem<kBf16>(src[int64_t(p + 2) * kD]);
      const float v2 = from_elem<kBf16>(src[int64_t(p + 4) * kD]);
      const float v3 = from_elem<kBf16>(src[int64_t(p + 6) * kD]);
      O[0] = fmaf(s_w[p], v0, O[0]);
      O[1] = fmaf(s_w[p + 2], v1, O[1]);
      O[0] = fmaf(s_w[p + 4], v2, O[0]);
      O[1] = fmaf(s_w[p + 6], v3, O[1]);
    }
    for (; p < n; p += 2) O[0] = fmaf(s_w[p], from_elem<kBf16>(src[int64_t(p) * kD]), O[0]);
  }
  // sum of weights over the workgroup, and the two halves' outputs
  for (int off = 32; off > 0; off >>= 1) S += __shfl_xor(S, off);
  __syncthreads();
  if ((tid & 63) == 0) s_part[tid >> 6] = S;
  s_o[r][d] = O[0] + O[1];
  __syncthreads();
  if (tid < kD) {
    const float tot = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const float o = s_o[0][tid] + s_o[1][tid];
    dst[tid] = uint16_t(to_elem<kBf16>(tot > 0.f ? o / tot : 0.f));
  }
}

template <int G, bool kBf16>
void launch_decode(const XDecodeArgs& a, bool v1, int parts, int hkv, int seqs, hipStream_t s) {
  if (v1) {
    xpacked_decode_kernel<G, kBf16, true, 4><<<dim3(hkv, seqs, 1), 256, 0, s>>>(a);
  } else {
    xpacked_decode_kernel<G, kBf16, false, kV2Waves>
        <<<dim3(hkv, seqs, parts), 64 * kV2Waves, 0, s>>>(a);
    xpacked_reduce_kernel<kBf16><<<dim3(hkv * G, seqs), kRedThreads, 0, s>>>(a);
  }
}

template <bool kBf16>
bool dispatch(int group, const XDecodeArgs& a, bool v1, int parts, int hkv, int seqs,
              hipStream_t s) {
  switch (group) {
    case 1: launch_decode<1, kBf16>(a, v1, parts, hkv, seqs, s); return true;
    case 2: launch_decode<2, kBf16>(a, v1, parts, hkv, seqs, s); return true;
    case 4: launch_decode<4, kBf16>(a, v1, parts, hkv, seqs, s); return true;
    case 8: launch_decode<8, kBf16>(a, v1, parts, hkv, seqs, s); return true;
    default: return false;
  }
}

int paged_attention(bool v1, void* out, float* exp_sums, float* max_logits, void* tmp_out,
                    int32_t max_num_partitions, const void* query, int64_t q_stride,
                    const void* key_cache, const void* value_cache, int32_t num_seqs,
                    int32_t num_heads, int32_t num_kv_heads, int32_t head_size, float scale,
                    const int32_t* block_tables, int64_t block_table_stride,
                    int32_t max_blocks_per_seq, const int32_t* seq_lens, int32_t block_size,
                    int32_t max_seq_len, int64_t num_blocks, int32_t dtype,
                    int64_t kv_block_stride, int64_t kv_head_stride, void* stream) {
  KVC_REQUIRE(num_seqs >= 0 && max_seq_len >= 0, KVC_ERR_INVALID_ARG, "negative size");
  if (num_seqs == 0) return ok();
  KVC_REQUIRE(out && query && key_cache && value_cache && block_tables && seq_lens,
              KVC_ERR_INVALID_ARG, "null pointer");
  KVC_REQUIRE(head_size == kD && block_size == kBlock, KVC_ERR_UNSUPPORTED,
              "x-packed attention supports head_size 128 and block_size 16");
  KVC_REQUIRE(dtype == KVC_DTYPE_FP16 || dtype == KVC_DTYPE_BF16, KVC_ERR_UNSUPPORTED,
              "dtype must be fp16 or bf16");
  KVC_REQUIRE(num_kv_heads > 0 && num_heads % num_kv_heads == 0, KVC_ERR_INVALID_ARG,
              "num_heads must be a multiple of num_kv_heads");
  const int group = num_heads / num_kv_heads;
  KVC_REQUIRE(num_blocks > 0 && max_blocks_per_seq >= 0 &&
                  block_table_stride >= max_blocks_per_seq,
              KVC_ERR_INVALID_ARG, "bad block table / num_blocks");
  KVC_REQUIRE(kv_head_stride >= int64_t(kD) * kBlock &&
                  kv_block_stride >= kv_head_stride * num_kv_heads,
              KVC_ERR_INVALID_ARG, "cache strides smaller than a head / block");
  KVC_REQUIRE(q_stride >= int64_t(num_heads) * kD, KVC_ERR_INVALID_ARG,
              "query stride smaller than num_heads * head_size");
  KVC_REQUIRE(aligned(query, 16) && aligned(key_cache, 16) && aligned(value_cache, 16) &&
                  aligned(out, 2) && q_stride % 8 == 0 && kv_block_stride % 8 == 0 &&
                  kv_head_stride % 8 == 0,
              KVC_ERR_ALIGNMENT, "query/cache pointers and strides must be 16-byte aligned");
  const int parts = (max_seq_len + kPart - 1) / kPart;
  KVC_REQUIRE(num_seqs <= 65535 && parts <= 65535, KVC_ERR_INVALID_ARG,
              "at most 65535 sequences and 65535 partitions per call");
  if (!v1) {
    KVC_REQUIRE(exp_sums && max_logits && tmp_out, KVC_ERR_INVALID_ARG,
                "v2 needs exp_sums, max_logits and tmp_out");
    KVC_REQUIRE(max_num_partitions >= parts, KVC_ERR_WORKSPACE,
                "v2 scratch holds " + std::to_string(max_num_partitions) +
                    " partitions, max_seq_len needs " + std::to_string(parts));
  }
  XDecodeArgs a;
  a.q = static_cast<const uint16_t*>(query);
  a.q_stride = q_stride;
  a.k_cache = static_cast<const uint16_t*>(key_cache);
  a.v_cache = static_cast<const uint16_t*>(value_cache);
  a.block_stride = kv_block_stride;
  a.head_stride = kv_head_stride;
  a.num_blocks = num_blocks;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.bt_cols = max_blocks_per_seq;
  a.seq_lens = seq_lens;
  a.num_kv_heads = num_kv_heads;
  a.max_parts = v1 ? 1 : max_num_partitions;
  a.grid_parts = parts;
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.exp_sums = exp_sums;
  a.max_logits = max_logits;
  a.tmp_out = static_cast<uint16_t*>(tmp_out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid_parts = std::max(parts, 1);
  const bool okd = dtype == KVC_DTYPE_BF16
                       ? dispatch<true>(group, a, v1, grid_parts, num_kv_heads, num_seqs, s)
                       : dispatch<false>(group, a, v1, grid_parts, num_kv_heads, num_seqs, s);
  KVC_REQUIRE(okd, KVC_ERR_UNSUPPORTED, "group (num_heads / num_kv_heads) must be 1, 2, 4 or 8");
  KVC_LAUNCH_CHECK();
  return ok();
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_reshape_and_cache_xpacked(
    const void* key, const void* value, void* key_cache, void* value_cache,
    const int64_t* slot_mapping, int64_t num_tokens, int32_t num_heads, int32_t head_size,
    int32_t block_size, int32_t x, int64_t num_blocks, int64_t key_token_stride,
    int64_t value_token_stride, int64_t cache_block_stride, int64_t cache_head_stride,
    int32_t* oob_count, void* stream) {
  KVC_REQUIRE(num_tokens >= 0, KVC_ERR_INVALID_ARG, "num_tokens < 0");
  if (num_tokens == 0) return ok();
  KVC_REQUIRE(key && value && key_cache && value_cache && slot_mapping, KVC_ERR_INVALID_ARG,
              "null pointer");
  KVC_REQUIRE(head_size == kD && block_size == kBlock && x == kX, KVC_ERR_UNSUPPORTED,
              "x-packed layout supports head_size 128, block_size 16 and x = 8 (2-byte types)");
  KVC_REQUIRE(num_heads > 0 && num_blocks > 0, KVC_ERR_INVALID_ARG, "non-positive shape");
  KVC_REQUIRE((num_tokens + kBlock - 1) / kBlock * num_heads < (int64_t(1) << 31),
              KVC_ERR_INVALID_ARG, "too many tokens");
  KVC_REQUIRE(key_token_stride >= int64_t(num_heads) * kD &&
                  value_token_stride >= int64_t(num_heads) * kD,
              KVC_ERR_INVALID_ARG, "source token stride smaller than a row");
  KVC_REQUIRE(cache_head_stride >= int64_t(kD) * kBlock &&
                  cache_block_stride >= cache_head_stride * num_heads,
              KVC_ERR_INVALID_ARG, "cache strides smaller than a head / block");
  KVC_REQUIRE(aligned(key, 16) && aligned(value, 16) && aligned(key_cache, 16) &&
                  aligned(value_cache, 16) && key_token_stride % 8 == 0 &&
                  value_token_stride % 8 == 0 && cache_block_stride % 8 == 0 &&
                  cache_head_stride % 8 == 0,
              KVC_ERR_ALIGNMENT, "key/value/cache pointers and strides must be 16-byte aligned");
  XAppendArgs a;
  a.key = static_cast<const uint16_t*>(key);
  a.value = static_cast<const uint16_t*>(value);
  a.key_cache = static_cast<uint16_t*>(key_cache);
  a.value_cache = static_cast<uint16_t*>(value_cache);
  a.slots = slot_mapping;
  a.key_stride = key_token_stride;
  a.value_stride = value_token_stride;
  a.block_stride = cache_block_stride;
  a.head_stride = cache_head_stride;
  a.num_slots = num_blocks * kBlock;
  a.num_tokens = num_tokens;
  a.num_heads = num_heads;
  a.oob_count = oob_count;
  xpacked_append_kernel<<<dim3(unsigned((num_tokens + kBlock - 1) / kBlock * num_heads)),
                          kThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
  KVC_LAUNCH_CHECK();
  return ok();
}

extern "C" int kvc_paged_attention_v1(
    void* out, const void* query, int64_t q_stride, const void* key_cache,
    const void* value_cache, int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_size, float scale, const int32_t* block_tables, int64_t block_table_stride,
    int32_t max_blocks_per_seq, const int32_t* seq_lens, int32_t block_size,
    int32_t max_seq_len, int64_t num_blocks, int32_t dtype, int64_t kv_block_stride,
    int64_t kv_head_stride, void* stream) {
  return paged_attention(true, out, nullptr, nullptr, nullptr, 1, query, q_stride, key_cache,
                         value_cache, num_seqs, num_heads, num_kv_heads, head_size, scale,
                         block_tables, block_table_stride, max_blocks_per_seq, seq_lens,
                         block_size, max_seq_len, num_blocks, dtype, kv_block_stride,
                         kv_head_stride, stream);
}

extern "C" int kvc_paged_attention_v2(
    void* out, float* exp_sums, float* max_logits, void* tmp_out, int32_t max_num_partitions,
    const void* query, int64_t q_stride, const void* key_cache, const void* value_cache,
    int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t head_size, float scale,
    const int32_t* block_tables, int64_t block_table_stride, int32_t max_blocks_per_seq,
    const int32_t* seq_lens, int32_t block_size, int32_t max_seq_len, int64_t num_blocks,
    int32_t dtype, int64_t kv_block_stride, int64_t kv_head_stride, void* stream) {
  return paged_attention(false, out, exp_sums, max_logits, tmp_out, max_num_partitions, query,
                         q_stride, key_cache, value_cache, num_seqs, num_heads, num_kv_heads,
                         head_size, scale, block_tables, block_table_stride, max_blocks_per_seq,
                         seq_lens, block_size, max_seq_len, num_blocks, dtype, kv_block_stride,
                         kv_head_stride, stream);
}
