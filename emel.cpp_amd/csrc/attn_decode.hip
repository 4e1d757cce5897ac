// Split-K flash-decode GQA attention over the paged pool (gfx950, wave64).
//
// Replaces the reference's paged decode route compute_attention
// (text/generator/detail.hpp:3153-3230) and its contiguous flash route
// (kernel/detail.hpp:5238-5291) with one kernel family:
//
//   grid = (split, KV-head group, sequence); a workgroup is one wave per KV
//   head of the group (8 for 8 KV heads), all walking the same pages of one
//   split of one sequence, so it streams whole pages.  Each wave serves the
//   G = n_head / n_head_kv query heads of its KV head from the rows it
//   loads (GQA sharing); the next tile's rows are loaded before the current
//   tile is used.  q is rounded to fp16 as round_q_for_nonflash does
//   (detail.hpp:2898-2903) and P to fp16 as the reference rounds its
//   probabilities (detail.hpp:3146-3149); the softmax is online, in fp32,
//   with a lazily moved reference max.
//
//   MFMA route (head_dim <= 256, G <= 4, pages holding whole wave tiles):
//   each 4-lane block of a wave holds 4 tokens of one 16-dim chunk; scores
//   S^T = K . Q^T and the output O^T += V^T . P^T run on 4x4x4 MFMA blocks
//   (fp16 operands; q8_0 bytes as exact fp16 values),
//   and each lane keeps one head's softmax and 16 output dims.
//   Scalar route (other shapes): a lane holds 16 dims of two tokens, scores
//   and P.V by v_dot2_f32_f16, a DPP sum over the row's lanes.
//
//   At the end each wave merges its token groups (halving exchanges) and
//   writes one partial (m, l, acc[D]) per (sequence, head, split), or the
//   output itself when a sequence has one split; a second kernel merges the
//   splits.  For 2 to 64 sequences the splits are balanced over the batch's
//   actual lengths.
//
// q8_0 pools keep their int8 values exact: biased fp16 (b + 1152) for the
// fp16 operands with the bias removed through the sums of q and of the
// weights; the block scales are applied to the scores and folded into the
// weights p * d_v, which enter the MFMA as an fp16 hi + lo pair.
#include <hip/hip_runtime.h>

#include <cmath>
#include <atomic>
#include <cstdlib>

#include "device_common.hpp"
#include "emelk.h"
#include "pool_layout.hpp"

namespace emelk {
namespace {

using namespace emelk::dev;

constexpr int k_max_wpb = 8;  // waves (KV heads) per workgroup
constexpr int k_max_split_pages = 1024;
// Register sets of tile rows kept in flight.  Measured on MI355X at the
// Llama-3-8B shape: 3 sets (246 VGPRs) stream no faster than 2 (214), and 4
// spill; a read-only walk of the same 64 KiB pages tops out at 6.76 TB/s,
// which 2 sets already reach within 5%.
constexpr int k_decode_nb = 2;
// q8_0 at head_dim 128 was first built with only the scores on MFMA
// (v_mfma_f32_16x16x32_f16 with rows = (32-value block, head)): correct, 15%
// fewer VALU instructions, but no faster (5.23 vs 5.20 TB/s), since the
// shuffles that sum the blocks and hand P to the V lanes lengthened each
// tile's dependent chain; the 4x4x4 block layout (scores and P.V both on
// MFMA, no hand-over) is what made it faster.  Scaling K to fp16 before the
// MFMA breaks the 2e-3 bar on the x20-outlier data, and so does rounding
// the P.V weights p * d_v once to fp16 on some shapes (the reference's own
// fp16 rounding of P already spends half the bar there).  Workgroups of 4 KV
// heads instead of 8 ran at 4.44 vs 5.51 TB/s there, and with 3 waves per
// SIMD (168 VGPRs, one tile set in flight) at 3.06.

// Waves per workgroup = KV heads per workgroup: min(n_head_kv, 8) when it
// divides n_head_kv, else 1.
inline int32_t waves_per_block(int32_t n_head_kv) {
  for (int32_t w = k_max_wpb; w > 1; w >>= 1) {
    if (n_head_kv % w == 0) return w;
  }
  return 1;
}

struct decode_params {
  pool_layout L;
  const uint8_t *k_pool;
  const uint8_t *v_pool;
  int32_t layer;
  const float *q;
  const int32_t *kv_lens;
  const uint16_t *tables;
  int32_t table_stride;
  float c;  // scale * log2(e): p = exp2((s - m) * c)
  int32_t tokens_per_split;
  int32_t max_splits;
  float *part_acc;  // [n_seq][n_head][max_splits][D]
  float *part_ml;   // [n_seq][n_head][max_splits][2]
  // Fused append (null new_k: none): the token at position kv_lens - 1 of
  // each sequence, rows new_k/new_v fp32 [n_seq][n_head_kv][D], is stored
  // into k_wr/v_wr (the same pools) and attended from registers.
  const float *new_k;
  const float *new_v;
  uint8_t *k_wr;
  uint8_t *v_wr;
  // One split per sequence (max_splits == 1): the kernel writes the
  // normalised output here and no combine kernel runs; else null.
  float *direct_out;
  // Row mode (per-row chunked prefill): "sequence" v is row v % rows of
  // sequence v / rows, attending to [0, row_q_start[v / rows] + v % rows]
  // through that sequence's block-table row; null otherwise.
  const int32_t *row_q_start;
  int32_t rows;
  // Balanced splits (1) or the host plan's fixed split size (0); the host
  // plan's split size in tiles bounds the balanced one.
  int32_t balanced;
  int32_t host_tiles;
  int32_t bt_shift;  // log2(block_tokens) when a power of two, else -1
};

// log2(block_tokens) when it is a power of two, else -1: the tile loops then
// find a token's page and row by shift and mask instead of a division.
inline int32_t pow2_shift(int32_t bt) {
  for (int32_t b = 0; b < 31; ++b) {
    if ((1 << b) == bt) return b;
  }
  return -1;
}

// Balanced split plan of a batch of n_seq <= 64 sequences, the same in every
// wave that computes it: lane i holds sequence i's length, its split count
// s_i and the index of its first split (exclusive prefix).  Splits are tb
// tiles of `tile` tokens, tb = ceil(T / (cap - n_seq)) over the batch's T
// tiles, clamped to [1, host_tiles]; then sum s_i <= T / tb + n_seq <= cap
// (or, at tb = host_tiles, <= n_seq * ceil(max tiles / host_tiles) = cap),
// so every split has a workgroup of the grid and a workspace slot.
// Inclusive prefix sum over the wave by DPP: shifts of 1, 2, 4 and 8 lanes
// inside each 16-lane row, then lane 15 of a row into the next row and lane
// 31 into the upper half (row_bcast:15 / row_bcast:31).
__device__ __forceinline__ int32_t wave_scan_incl(int32_t x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15, rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31, rows 2 and 3
  return x;
}

__device__ __forceinline__ void balanced_splits(const int32_t *__restrict__ kv_lens, int32_t n_seq,
                                                int32_t cap, int32_t host_tiles, int32_t tile,
                                                int32_t lane, int32_t &len_i, int32_t &s_i,
                                                int32_t &excl_i, int32_t &tb) {
  len_i = lane < n_seq ? kv_lens[lane] : 0;
  const int32_t t_i = len_i > 0 ? (len_i + tile - 1) / tile : 0;
  const int32_t incl = wave_scan_incl(t_i);
  const int32_t T = __builtin_amdgcn_readlane(incl, k_wave - 1);
  tb = cap > n_seq ? (T + (cap - n_seq) - 1) / (cap - n_seq) : host_tiles;
  tb = tb < 1 ? 1 : (tb > host_tiles ? host_tiles : tb);
  s_i = (t_i + tb - 1) / tb;
  excl_i = wave_scan_incl(s_i) - s_i;
}


// 16 int8 -> 8 half2 holding b + 1152 exactly: byte b becomes the fp16 bit
// pattern 0x64XX with XX = b + 128, whose value is 1024 + b + 128.  The
// constant 1152 is removed from the dot product by starting it at
// -1152 * (sum of the lane's q values), so no per-value subtract is needed.
__device__ __forceinline__ void i8x16_to_half_biased(const uint4_t w, half2_t out[8]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = ws[i] ^ 0x80808080u;
    out[2 * i] = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
    out[2 * i + 1] = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
  }
}

// Two rows of 16 int8 (tokens t0, t1, same dims) -> 16 half2 pairs
// (q_t0[i] + 1152, q_t1[i] + 1152), exact: one permute interleaves two dims
// of both tokens, two permutes put each byte (biased by +128) under the
// fp16 exponent of 1024.  The constant 1152 stays in the products; the
// decode subtracts 1152 times the sum of its fp16 P.V weights at the end
// (measured 2% faster than a packed fp16 add per pair).
__device__ __forceinline__ void i8x16_pair_to_half2(const uint4_t w0, const uint4_t w1,
                                                    half2_t out[16]) {
  const uint32_t a[4] = {w0.x ^ 0x80808080u, w0.y ^ 0x80808080u, w0.z ^ 0x80808080u,
                         w0.w ^ 0x80808080u};
  const uint32_t b[4] = {w1.x ^ 0x80808080u, w1.y ^ 0x80808080u, w1.z ^ 0x80808080u,
                         w1.w ^ 0x80808080u};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // bytes (a0, b0, a1, b1) and (a2, b2, a3, b3)
    const uint32_t lo = __builtin_amdgcn_perm(b[i], a[i], 0x05010400u);
    const uint32_t hi = __builtin_amdgcn_perm(b[i], a[i], 0x07030602u);
    out[4 * i + 0] = as_half2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u));
    out[4 * i + 1] = as_half2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u));
    out[4 * i + 2] = as_half2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u));
    out[4 * i + 3] = as_half2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u));
  }
}

// (x0, x1) as fp16 pairs hi + lo: hi = fp16(x), lo = fp16(x - hi), so hi + lo
// carries x to about 2^-22 relative (|x| in the fp16 normal range; below it
// to the fp16 subnormal step).  The q8_0 P.V weights p * d_v go to the MFMA
// as both halves, so the output sees them at nearly fp32 accuracy.
__device__ __forceinline__ void split_half2(float x0, float x1, half2_t &hi, half2_t &lo) {
  hi = pack_half2(x0, x1);
  lo = pack_half2(x0 - static_cast<float>(hi.x), x1 - static_cast<float>(hi.y));
}

template <int D, bool Q8>
struct row_regs;
template <int D>
struct row_regs<D, false> {
  uint4_t a, b;  // 16 halves
};
template <int D>
struct row_regs<D, true> {
  uint4_t a;     // 16 int8
  uint32_t d;    // scale bits (low 16)
};

// Lane dims.  f16 rows (2*D bytes): the lane's 16 dims are two runs of 8,
// [8*l, 8*l+8) and [D/2 + 8*l, D/2 + 8*l + 8) for lane l of the row, so each
// load instruction of a wave covers whole contiguous half rows (full 128-byte
// lines at D = 128).  q8_0 rows (D bytes): one run [16*l, 16*l + 16).
template <int D, bool Q8>
__device__ __forceinline__ int lane_dim(int lane_in_row, int i) {
  if constexpr (Q8) {
    return 16 * lane_in_row + i;
  } else {
    return (i < 8 ? 0 : D / 2 - 8) + 8 * lane_in_row + i;
  }
}

template <int D, bool Q8>
__device__ __forceinline__ void load_row(const uint8_t *__restrict__ region_base, int32_t off,
                                         int32_t lane_in_row, int32_t bt, row_regs<D, Q8> &r) {
  if constexpr (!Q8) {
    const uint8_t *p = region_base + static_cast<uint64_t>(off) * D * 2u + lane_in_row * 16;
    r.a = load16_stream(p);
    r.b = load16_stream(p + D);
  } else {
    const int32_t dim0 = 16 * lane_in_row;
    r.a = load16_stream(region_base + static_cast<uint64_t>(off) * D + dim0);
    const uint16_t *sc = reinterpret_cast<const uint16_t *>(region_base + static_cast<uint64_t>(bt) * D);
    r.d = load2_stream(sc + off * (D / 32) + dim0 / 32);
  }
}

// Same rows, addressed as a wave-uniform base plus a fixed per-lane 32-bit
// offset, so the loads take the scalar-base form and need no per-lane 64-bit
// address arithmetic.  `region` is the (page, head) region, `row0` the
// page offset of the wave's first row (both uniform); `lane_off` and
// `lane_sc_off` are the lane's byte offsets of its values and of its q8_0
// block scale relative to that row.
template <int D, bool Q8>
__device__ __forceinline__ void load_row_uniform(const uint8_t *__restrict__ region, int32_t row0,
                                                 uint32_t lane_off, uint32_t lane_sc_off,
                                                 int32_t bt, row_regs<D, Q8> &r) {
  if constexpr (!Q8) {
    const uint8_t *u = region + static_cast<uint32_t>(row0) * (2u * D);
    r.a = load16_stream(u + lane_off);
    r.b = load16_stream(u + lane_off + D);
  } else {
    const uint8_t *u = region + static_cast<uint32_t>(row0) * static_cast<uint32_t>(D);
    r.a = load16_stream(u + lane_off);
    const uint8_t *s = region + static_cast<uint32_t>(bt) * D + static_cast<uint32_t>(row0) * (D / 16);
    r.d = load2_stream(s + lane_sc_off);
  }
}

// The stored form of one new row, in the lane layout of row_regs: f16 pools
// round to fp16 (fp32_to_fp16, kernel/detail.hpp:372-392); q8_0 pools
// quantize each 32-value block as quantize_row_q8_0_strided
// (kernel/detail.hpp:804-824), the two lanes of a block sharing its amax.
template <int D, bool Q8>
__device__ __forceinline__ void new_row_regs(const float *__restrict__ row, int32_t lane_in_row,
                                             int32_t block_partner, row_regs<D, Q8> &r) {
  if constexpr (!Q8) {
    const float4_t a0 = *reinterpret_cast<const float4_t *>(row + 8 * lane_in_row);
    const float4_t a1 = *reinterpret_cast<const float4_t *>(row + 8 * lane_in_row + 4);
    const float4_t b0 = *reinterpret_cast<const float4_t *>(row + D / 2 + 8 * lane_in_row);
    const float4_t b1 = *reinterpret_cast<const float4_t *>(row + D / 2 + 8 * lane_in_row + 4);
    r.a = uint4_t{as_u32(pack_half2(a0.x, a0.y)), as_u32(pack_half2(a0.z, a0.w)),
                  as_u32(pack_half2(a1.x, a1.y)), as_u32(pack_half2(a1.z, a1.w))};
    r.b = uint4_t{as_u32(pack_half2(b0.x, b0.y)), as_u32(pack_half2(b0.z, b0.w)),
                  as_u32(pack_half2(b1.x, b1.y)), as_u32(pack_half2(b1.z, b1.w))};
  } else {
    float v[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4_t f = *reinterpret_cast<const float4_t *>(row + 16 * lane_in_row + 4 * j);
      v[4 * j + 0] = f.x;
      v[4 * j + 1] = f.y;
      v[4 * j + 2] = f.z;
      v[4 * j + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, block_partner, k_wave));  // the other half of the block
    const float d = amax / 127.0f;
    const float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      int q = static_cast<int>(roundf(v[j] * inv_d));
      q = q < -127 ? -127 : (q > 127 ? 127 : q);
      w[j / 4] |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * (j % 4));
    }
    r.a = uint4_t{w[0], w[1], w[2], w[3]};
    r.d = f32_to_f16_bits(d);
  }
}

template <int D, bool Q8>
__device__ __forceinline__ void to_half(const row_regs<D, Q8> &r, half2_t h[8], float &scale) {
  if constexpr (!Q8) {
    const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = as_half2(w[j]);
    scale = 1.0f;
  } else {
    i8x16_to_half_biased(r.a, h);
    scale = f16_bits_to_f32(static_cast<uint16_t>(r.d));
  }
}

// Lazy rescaling: the running reference max of a head only moves when a
// score exceeds it by more than k_rescale (log2 units), so exp2(y - m) stays
// <= 2^k_rescale (fine for fp32 sums and for the fp16 P operand) and the
// accumulator rescale is skipped on almost every tile.  Any reference value
// gives the same softmax once l and acc are merged against it.
constexpr float k_rescale = 8.0f;

template <int D, int G, bool Q8>
struct decode_state {
  half2_t qh[G][8];  // fp16 q, 16 dims of each head
  float m[G];        // reference max (log2 domain, scale folded in)
  float l[G];
  float acc[G][16];
  float kbias[G];    // q8_0: -1152 * sum of the lane's 16 q values (K byte bias)
  float vw[G];       // q8_0: sum of the fp16 P.V weights (V byte bias 1152 removed at the end)
  // scores on MFMA: fp16 q of head 4 * set + lane % 4 over the lane's 16
  // dims, in four 4-dim steps (the K row's order), zero past G
  half4_t qm[(G + 3) / 4][4];
  // q8_0 MPV route: the K byte bias of the lane's own head of each set
  float kb[(G + 3) / 4];
};

template <int D, bool Q8>
struct tile_regs {
  row_regs<D, Q8> k0, k1, v0, v1;
};

// One tile: two tokens per lane group (t0, t1).  MASKED handles the split's
// tail and invalid pages (ok0/ok1 false).
template <int D, int G, bool Q8, bool MASKED, bool MQK>
__device__ __forceinline__ void consume_tile(decode_state<D, G, Q8> &S, const tile_regs<D, Q8> &T,
                                             bool ok0, bool ok1, float c) {
  constexpr int LPT = D / 16;
  float y0[G], y1[G];
  if constexpr (MQK) {
    // q8_0 scores on v_mfma_f32_4x4x4_16b_f16: each 4-lane block holds 4
    // tokens (B columns: the K bytes as exact fp16 b + 1152) of one 16-dim
    // chunk and the exact fp16 q of 4 heads (A rows); lane 4b+j receives the
    // 4 heads' sums for its token j over the chunk.  Each accumulator starts
    // at the head's -1152 * sum q, which removes the byte bias.
    static_assert(Q8, "MFMA scores on this route need q8_0 keys");
    half2_t kh0[8], kh1[8];
    i8x16_to_half_biased(T.k0.a, kh0);
    i8x16_to_half_biased(T.k1.a, kh1);
    const float ks0 = f16_bits_to_f32(static_cast<uint16_t>(T.k0.d)) * c;
    const float ks1 = f16_bits_to_f32(static_cast<uint16_t>(T.k1.d)) * c;
#pragma unroll
    for (int g4 = 0; g4 < (G + 3) / 4; ++g4) {
      float4_t a0;
#pragma unroll
      for (int r = 0; r < 4; ++r) a0[r] = 4 * g4 + r < G ? S.kbias[4 * g4 + r < G ? 4 * g4 + r : 0] : 0.0f;
      float4_t a1 = a0;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const half4_t k0 = {kh0[2 * m].x, kh0[2 * m].y, kh0[2 * m + 1].x, kh0[2 * m + 1].y};
        const half4_t k1 = {kh1[2 * m].x, kh1[2 * m].y, kh1[2 * m + 1].x, kh1[2 * m + 1].y};
        a0 = __builtin_amdgcn_mfma_f32_4x4x4f16(S.qm[g4][m], k0, a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_f32_4x4x4f16(S.qm[g4][m], k1, a1, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = 4 * g4 + r;
        if (h < G) {
          y0[h] = chunk_sum<LPT>(a0[r] * ks0);
          y1[h] = chunk_sum<LPT>(a1[r] * ks1);
          if constexpr (MASKED) {
            y0[h] = ok0 ? y0[h] : -INFINITY;
            y1[h] = ok1 ? y1[h] : -INFINITY;
          }
        }
      }
    }
  } else {
  half2_t kh0[8], kh1[8];
  float ks0, ks1;
  to_half<D, Q8>(T.k0, kh0, ks0);
  to_half<D, Q8>(T.k1, kh1, ks1);
  if constexpr (Q8) {  // the softmax scale folds into each token's block scale
    ks0 *= c;
    ks1 *= c;
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float a = Q8 ? S.kbias[h] : 0.0f;
    float b = a;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a = dot2(S.qh[h][j], kh0[j], a);
      b = dot2(S.qh[h][j], kh1[j], b);
    }
    if constexpr (Q8) {  // each lane's 16 values share one block scale
      y0[h] = group_sum<LPT>(a * ks0);
      y1[h] = group_sum<LPT>(b * ks1);
    } else {
      y0[h] = group_sum<LPT>(a) * c;
      y1[h] = group_sum<LPT>(b) * c;
    }
    if constexpr (MASKED) {
      y0[h] = ok0 ? y0[h] : -INFINITY;
      y1[h] = ok1 ? y1[h] : -INFINITY;
    }
  }
  }

  // V operands: both pools pair the two tokens per dimension for
  // v_dot2_f32_f16: f16 pools with the fp16 pair (p0, p1), q8_0 pools with
  // the exact fp16 q values and the pair (p0 * d_v0, p1 * d_v1).
  [[maybe_unused]] half2_t vlo[8], vhi[8];
  [[maybe_unused]] half2_t vq[16];
  [[maybe_unused]] float vs0 = 1.0f, vs1 = 1.0f;
  // Masked tokens (past the end, invalid page) were read from a clamped
  // address that may hold never-written bytes: their V words and scales are
  // zeroed, since p = 0 times a NaN slot would still be NaN.
  if constexpr (!Q8) {
    uint32_t w0[8] = {T.v0.a.x, T.v0.a.y, T.v0.a.z, T.v0.a.w,
                      T.v0.b.x, T.v0.b.y, T.v0.b.z, T.v0.b.w};
    uint32_t w1[8] = {T.v1.a.x, T.v1.a.y, T.v1.a.z, T.v1.a.w,
                      T.v1.b.x, T.v1.b.y, T.v1.b.z, T.v1.b.w};
    if constexpr (MASKED) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        w0[j] = ok0 ? w0[j] : 0u;
        w1[j] = ok1 ? w1[j] : 0u;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      vlo[j] = as_half2(__builtin_amdgcn_perm(w1[j], w0[j], 0x05040100u));
      vhi[j] = as_half2(__builtin_amdgcn_perm(w1[j], w0[j], 0x07060302u));
    }
  } else {
    i8x16_pair_to_half2(T.v0.a, T.v1.a, vq);
    vs0 = f16_bits_to_f32(static_cast<uint16_t>(T.v0.d));
    vs1 = f16_bits_to_f32(static_cast<uint16_t>(T.v1.d));
    if constexpr (MASKED) {  // the int8 values are always finite
      vs0 = ok0 ? vs0 : 0.0f;
      vs1 = ok1 ? vs1 : 0.0f;
    }
  }

#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float mx = fmaxf(y0[h], y1[h]);
    if (mx > S.m[h] + k_rescale) {
      const float alpha = fast_exp2(S.m[h] - mx);  // 0 on the first valid token
      S.m[h] = mx;
      S.l[h] *= alpha;
      if constexpr (Q8) S.vw[h] *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) S.acc[h][i] *= alpha;
    }
    float p0 = fast_exp2(y0[h] - S.m[h]);
    float p1 = fast_exp2(y1[h] - S.m[h]);
    if constexpr (MASKED) {  // masked tokens, also while m is still -inf
      p0 = y0[h] == -INFINITY ? 0.0f : p0;
      p1 = y1[h] == -INFINITY ? 0.0f : p1;
    }
    S.l[h] += p0 + p1;
    if constexpr (Q8) {
      // weights p * d_v as fp16 hi + lo pairs against the exact fp16 values
      half2_t wh, wl;
      split_half2(p0 * vs0, p1 * vs1, wh, wl);
#pragma unroll
      for (int i = 0; i < 16; ++i) S.acc[h][i] = dot2(wl, vq[i], dot2(wh, vq[i], S.acc[h][i]));
      S.vw[h] = dot2(wl, as_half2(0x3C003C00u), dot2(wh, as_half2(0x3C003C00u), S.vw[h]));
    } else {
      const half2_t pp = pack_half2(p0, p1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        S.acc[h][2 * j] = dot2(pp, vlo[j], S.acc[h][2 * j]);
        S.acc[h][2 * j + 1] = dot2(pp, vhi[j], S.acc[h][2 * j + 1]);
      }
    }
  }
}

// MPV tile (MFMA lane layout): scores and P.V both on 4x4x4 MFMA blocks,
// each 4-lane block holding 4 tokens of one 16-dim chunk, one set of 4
// query heads per pass (two sets at G = 8, lane j serving heads j, j + 4).
//   scores  S^T (4 tokens x 4 heads) = K (4 x 16 dims) . Q^T   (4 steps of 4 dims)
//   output  O^T (4 dims x 4 heads)  += V^T (4 dims x 4 tokens) . P'^T
// so lane 4b+j ends each step with head j: its 4 tokens' scores, then its
// 16 dims of O over the block's tokens, and the softmax runs per lane for
// one head.  T.k{0,1} hold the lane's own token row (token j + 4q of each
// half); T.v{0,1} hold 4 dims of the chunk (mpv_dim) for the block's 4
// tokens.
//   q8_0: K bytes as exact fp16 values b + 1152 on v_mfma_f32_4x4x4_16b_f16
//   against the fp16 q (each accumulator starts at the lane's head's -1152 *
//   sum q, which removes the bias), scaled by the token's K block scale
//   (from the lane that loaded it); V.d is the lane's own token's V block
//   scale, P' = p * d_v of each token (the lane's 16 dims lie in one scale
//   block) as an fp16 hi + lo pair (two MFMAs), and the V bytes enter as
//   the exact fp16 values b + 1152 (the 1152 * sum P' term is removed at the
//   end through vw).
//   f16: K halves on v_mfma_f32_4x4x4_16b_f16 against q in fp16; P' = p;
//   V.a holds tokens 0 and 1 (two words each), V.b tokens 2 and 3.
// ok0/ok1: the lane's own token is valid.
template <int D, bool Q8>
__device__ __forceinline__ int mpv_dim(int chunk, int j) {  // first of the lane's 4 dims
  if constexpr (Q8) {
    return 16 * chunk + 4 * j;
  } else {  // the chunk's two runs of 8 (lane_dim): j = 0, 1 in the first
    return (j < 2 ? 0 : D / 2) + 8 * chunk + 4 * (j & 1);
  }
}

template <int D, int G, bool Q8, bool MASKED>
__device__ __forceinline__ void consume_tile_mpv(decode_state<D, G, Q8> &S,
                                                 const tile_regs<D, Q8> &T, bool ok0, bool ok1,
                                                 float c) {
  constexpr int LPT = D / 16;
  constexpr int NHS = (G + 3) / 4;  // head sets: lane j serves heads j and j + 4
  float y[NHS][2][4];
  [[maybe_unused]] float dk_b[2][4];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const row_regs<D, Q8> &K = hf == 0 ? T.k0 : T.k1;
    if constexpr (Q8) {
      // token i's K block scale comes from lane i of the block
      const float dk = f16_bits_to_f32(static_cast<uint16_t>(K.d)) * c;
      dk_b[hf][0] = quad_bcast<0>(dk);
      dk_b[hf][1] = quad_bcast<1>(dk);
      dk_b[hf][2] = quad_bcast<2>(dk);
      dk_b[hf][3] = quad_bcast<3>(dk);
    }
    // K operand of step m (dims 4m .. 4m + 3 of the chunk), fp16; q8_0 bytes
    // as exact fp16 b + 1152, the bias removed by the accumulator's start
    half4_t ka[4];
    if constexpr (Q8) {
      half2_t kh[8];
      i8x16_to_half_biased(K.a, kh);
#pragma unroll
      for (int m = 0; m < 4; ++m) ka[m] = half4_t{kh[2 * m].x, kh[2 * m].y, kh[2 * m + 1].x, kh[2 * m + 1].y};
    } else {
      const uint32_t kw[8] = {K.a.x, K.a.y, K.a.z, K.a.w, K.b.x, K.b.y, K.b.z, K.b.w};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const half2_t k01 = as_half2(kw[2 * m]), k23 = as_half2(kw[2 * m + 1]);
        ka[m] = half4_t{k01.x, k01.y, k23.x, k23.y};
      }
    }
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      const float s0 = Q8 ? S.kb[hs] : 0.0f;
      float4_t sc = {s0, s0, s0, s0};
#pragma unroll
      for (int m = 0; m < 4; ++m) sc = __builtin_amdgcn_mfma_f32_4x4x4f16(ka[m], S.qm[hs][m], sc, 0, 0, 0);
      if constexpr (Q8) {  // token i's K block scale (softmax scale folded in)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[hs][hf][i] = chunk_sum<LPT>(sc[i] * dk_b[hf][i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) y[hs][hf][i] = chunk_sum<LPT>(sc[i]) * c;
      }
    }
    if constexpr (MASKED) {
      const float okf = (hf == 0 ? ok0 : ok1) ? 1.0f : 0.0f;
      const float ok_b[4] = {quad_bcast<0>(okf), quad_bcast<1>(okf), quad_bcast<2>(okf),
                             quad_bcast<3>(okf)};
#pragma unroll
      for (int hs = 0; hs < NHS; ++hs) {
#pragma unroll
        for (int i = 0; i < 4; ++i) y[hs][hf][i] = ok_b[i] != 0.0f ? y[hs][hf][i] : -INFINITY;
      }
    }
  }
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs) {
    float mx = y[hs][0][0];
#pragma unroll
    for (int k = 1; k < 8; ++k) mx = fmaxf(mx, y[hs][k / 4][k % 4]);
    if (mx > S.m[hs] + k_rescale) {
      const float alpha = fast_exp2(S.m[hs] - mx);  // 0 on the first valid token
      S.m[hs] = mx;
      S.l[hs] *= alpha;
      if constexpr (Q8) S.vw[hs] *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) S.acc[hs][i] *= alpha;
    }
  }
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const row_regs<D, Q8> &V = hf == 0 ? T.v0 : T.v1;
    half4_t va[4];  // A operand of dim s: its value for the block's tokens 0..3
    [[maybe_unused]] float dv_b[4];
    if constexpr (Q8) {
      float dv = f16_bits_to_f32(static_cast<uint16_t>(V.d));
      if constexpr (MASKED) dv = (hf == 0 ? ok0 : ok1) ? dv : 0.0f;  // a masked slot may hold NaN bits
      dv_b[0] = quad_bcast<0>(dv);
      dv_b[1] = quad_bcast<1>(dv);
      dv_b[2] = quad_bcast<2>(dv);
      dv_b[3] = quad_bcast<3>(dv);
      const uint32_t w0 = V.a.x ^ 0x80808080u, w1 = V.a.y ^ 0x80808080u;
      const uint32_t w2 = V.a.z ^ 0x80808080u, w3 = V.a.w ^ 0x80808080u;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        // bytes of dims 2*s2 and 2*s2+1 of tokens (0, 1) and (2, 3)
        const uint32_t sel = s2 == 0 ? 0x05010400u : 0x07030602u;
        const uint32_t x01 = __builtin_amdgcn_perm(w1, w0, sel);
        const uint32_t x23 = __builtin_amdgcn_perm(w3, w2, sel);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const uint32_t cs = e == 0 ? 0x04010400u : 0x04030402u;
          const half2_t a01 = as_half2(__builtin_amdgcn_perm(0x64646464u, x01, cs));
          const half2_t a23 = as_half2(__builtin_amdgcn_perm(0x64646464u, x23, cs));
          va[2 * s2 + e] = half4_t{a01.x, a01.y, a23.x, a23.y};
        }
      }
    } else {
      // token t's dims (0, 1) in word 2t, (2, 3) in word 2t + 1 (a: t = 0, 1; b: t = 2, 3)
      uint32_t tw[8] = {V.a.x, V.a.y, V.a.z, V.a.w, V.b.x, V.b.y, V.b.z, V.b.w};
      if constexpr (MASKED) {  // masked slots may hold NaN bits: p = 0 would not clear them
        const float okf = (hf == 0 ? ok0 : ok1) ? 1.0f : 0.0f;
        const float ok_b[4] = {quad_bcast<0>(okf), quad_bcast<1>(okf), quad_bcast<2>(okf),
                               quad_bcast<3>(okf)};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          tw[2 * t] = ok_b[t] != 0.0f ? tw[2 * t] : 0u;
          tw[2 * t + 1] = ok_b[t] != 0.0f ? tw[2 * t + 1] : 0u;
        }
      }
#pragma unroll
      for (int sd = 0; sd < 4; ++sd) {
        const int wi = sd / 2;                                // word of the dim
        const uint32_t sel = sd % 2 == 0 ? 0x05040100u : 0x07060302u;  // its half
        const half2_t a01 = as_half2(__builtin_amdgcn_perm(tw[2 + wi], tw[wi], sel));
        const half2_t a23 = as_half2(__builtin_amdgcn_perm(tw[6 + wi], tw[4 + wi], sel));
        va[sd] = half4_t{a01.x, a01.y, a23.x, a23.y};
      }
    }
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = fast_exp2(y[hs][hf][i] - S.m[hs]);
        if constexpr (MASKED) p[i] = y[hs][hf][i] == -INFINITY ? 0.0f : p[i];
      }
      S.l[hs] += (p[0] + p[1]) + (p[2] + p[3]);
      half4_t pw;
      [[maybe_unused]] half4_t pl;
      if constexpr (Q8) {  // P' = p * d_v as fp16 hi (pw) + lo (pl)
        half2_t h01, l01, h23, l23;
        split_half2(p[0] * dv_b[0], p[1] * dv_b[1], h01, l01);
        split_half2(p[2] * dv_b[2], p[3] * dv_b[3], h23, l23);
        const half2_t one = as_half2(0x3C003C00u);
        S.vw[hs] = dot2(l23, one, dot2(h23, one, dot2(l01, one, dot2(h01, one, S.vw[hs]))));
        pw = half4_t{h01.x, h01.y, h23.x, h23.y};
        pl = half4_t{l01.x, l01.y, l23.x, l23.y};
      } else {
        const half2_t w01 = pack_half2(p[0], p[1]);
        const half2_t w23 = pack_half2(p[2], p[3]);
        pw = half4_t{w01.x, w01.y, w23.x, w23.y};
      }
#pragma unroll
      for (int sd = 0; sd < 4; ++sd) {  // dim sd of the lane's 4 in output register i = lane i's
        float4_t o = {S.acc[hs][4 * sd], S.acc[hs][4 * sd + 1], S.acc[hs][4 * sd + 2],
                      S.acc[hs][4 * sd + 3]};
        o = __builtin_amdgcn_mfma_f32_4x4x4f16(va[sd], pw, o, 0, 0, 0);
        if constexpr (Q8) o = __builtin_amdgcn_mfma_f32_4x4x4f16(va[sd], pl, o, 0, 0, 0);
        S.acc[hs][4 * sd] = o.x;
        S.acc[hs][4 * sd + 1] = o.y;
        S.acc[hs][4 * sd + 2] = o.z;
        S.acc[hs][4 * sd + 3] = o.w;
      }
    }
  }
}

template <int D, int G, bool Q8, bool MASKED, bool MQK, bool MPV>
__device__ __forceinline__ void consume_any(decode_state<D, G, Q8> &S, const tile_regs<D, Q8> &T,
                                            bool ok0, bool ok1, float c) {
  if constexpr (MPV) {
    consume_tile_mpv<D, G, Q8, MASKED>(S, T, ok0, ok1, c);
  } else {
    consume_tile<D, G, Q8, MASKED, MQK>(S, T, ok0, ok1, c);
  }
}

// Workgroup = WPB waves = WPB KV heads of one sequence over one split of
// its context; wave w owns KV head blockIdx.y*WPB + w and its G query heads.
// All waves walk the same pages at the same time, so a workgroup reads
// whole pages (every head's slice) rather than one 8 KiB head slice per
// page: measured on MI355X this access order streams ~15% faster from HBM.
// Each wave merges its own token groups with shuffles; no cross-wave step.
//
// UNIFORM: block_tokens is a multiple of the wave's lane-group count NGW, so
// every row of a (tile, half) lies in one page: the page id is moved to a
// scalar register once per half-tile and each lane adds a fixed offset.
//
// MQK (q8_0, head_dim <= 256): scores on 4x4x4 MFMA.  The lane layout
// then puts the 4 tokens of an MFMA block in lane bits 0-1 and the 16-dim
// chunk in the bits above them: lane = j + 4 * chunk + 4 * LPT * q holds
// chunk `chunk` of token j + 4 * q of each half-tile.
//
// MPV (MQK with UNIFORM): P.V on MFMA as well (consume_tile_mpv); a lane
// serves one query head per set of 4 (two sets at G = 8).
template <int D, int G, bool Q8, bool UNIFORM, int WPB, int NB, bool MQK, bool MPV>
__global__ __launch_bounds__(WPB * k_wave) void decode_kernel(decode_params P) {
  static_assert(!MPV || (MQK && UNIFORM && G <= 8), "MPV layout");
  constexpr int LPT = D / 16;         // lanes per token row
  constexpr int NGW = k_wave / LPT;   // token groups per wave
  constexpr int TT = 2 * NGW;         // tokens per wave tile
  constexpr int NT = WPB * k_wave;
  constexpr uint32_t ROWB = Q8 ? D : 2 * D;  // bytes of one K/V row in a page

  __shared__ uint32_t s_pages[k_max_split_pages];

  const int32_t tid = threadIdx.x;
  // the wave index is uniform; readfirstlane lets the compiler keep the
  // head's base pointers in scalar registers
  const int32_t wave = __builtin_amdgcn_readfirstlane(tid / k_wave);
  const int32_t lane = tid % k_wave;
  const int32_t kvh = blockIdx.y * WPB + wave;
  // Start-up in one round trip: the length, q and the split's page-table
  // entries are all requested before any of them is used (the page count
  // of a split is bounded by tokens_per_split, so the entries are read
  // before the length is known).
  // With balanced splits the workgroup first reads every length of the
  // batch (one more round trip) and takes split w = blockIdx.x + gridDim.x *
  // blockIdx.z of the balanced plan.  Partial of head h: row slot_base + h *
  // slot_stride of the workspace.
  int32_t seq = blockIdx.z;
  int32_t split = blockIdx.x;
  int32_t tps = P.tokens_per_split;
  int32_t len;
  uint64_t slot_base;
  uint32_t slot_stride;
  if (P.balanced) {
    const int32_t w = blockIdx.x + gridDim.x * blockIdx.z;
    int32_t len_i, s_i, excl_i, tb;
    balanced_splits(P.kv_lens, gridDim.z, gridDim.x * gridDim.z, P.host_tiles, TT, lane, len_i,
                    s_i, excl_i, tb);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(s_i > 0 && excl_i <= w && w < excl_i + s_i);
    if (hit == 0) return;  // uniform: more workgroups than splits
    seq = __builtin_ctzll(hit);
    split = w - __builtin_amdgcn_readlane(excl_i, seq);
    len = __builtin_amdgcn_readlane(len_i, seq);
    tps = tb * TT;
    slot_base = static_cast<uint64_t>(w) * P.L.n_head + kvh * G;
    slot_stride = 1u;
  } else {
    if (P.row_q_start != nullptr) {  // a negative chunk start attends to nothing (zero rows)
      const int32_t q0 = P.row_q_start[seq / P.rows];
      len = q0 < 0 ? 0 : q0 + (seq % P.rows) + 1;
    } else {
      len = P.kv_lens[seq];
    }
    slot_base = (static_cast<uint64_t>(seq) * P.L.n_head + kvh * G) * P.max_splits + split;
    slot_stride = static_cast<uint32_t>(P.max_splits);
  }
  const int32_t table_row = P.row_q_start != nullptr ? seq / P.rows : seq;
  const int32_t start = split * tps;
  const int32_t bt = P.L.block_tokens;
  const int32_t first_page = start / bt;
  // lane_in_row: the lane's 16-dim chunk of a row; grp: its token of a
  // half-tile
  const int32_t lane_in_row = MQK ? (lane >> 2) % LPT : lane % LPT;
  const int32_t grp = MQK ? (lane & 3) + 4 * (lane / (4 * LPT)) : lane / LPT;
  // lane distance to the other 16 dims of a q8_0 block, and to the lanes of
  // the same dims in the token groups merged at the end (bit r of grp)
  constexpr int block_partner = MQK ? 4 : 1;
  auto grp_mask = [](int r) { return MQK ? (r < 2 ? 1 << r : LPT << r) : LPT << r; };
  float4_t qraw[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float *qp = P.q + (static_cast<uint64_t>(seq) * P.L.n_head + kvh * G + h) * D;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qraw[h][j] = *reinterpret_cast<const float4_t *>(qp + lane_dim<D, Q8>(lane_in_row, 4 * j));
    }
  }
  constexpr int PPT = (k_max_split_pages + NT - 1) / NT;  // page entries per thread
  const int32_t max_pages = min(k_max_split_pages, P.tokens_per_split / bt + 2);
  // Null tables: contiguous caches, page = table_row * table_stride + block
  // (no table read between the start and the first tile's loads).
  const bool contiguous = P.tables == nullptr;
  const uint64_t table_base = static_cast<uint64_t>(table_row) * P.table_stride;
  const uint16_t *table = contiguous ? nullptr : P.tables + table_base;
  uint32_t pg[PPT];
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int32_t i = tid + k * NT;
    const int32_t lb = first_page + i;
    pg[k] = (i < max_pages && lb < P.table_stride)
                ? (contiguous ? static_cast<uint32_t>(table_base + lb) : table[lb])
                : 0xFFFFFFFFu;
  }
  if (start >= len) {  // uniform; the combine kernel never reads this split
    if (P.direct_out != nullptr && grp == 0) {  // nothing to attend: zero output
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float *op = P.direct_out + (static_cast<uint64_t>(seq) * P.L.n_head + kvh * G + h) * D;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          *reinterpret_cast<float4_t *>(op + lane_dim<D, Q8>(lane_in_row, 4 * j)) =
              float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
    }
    return;
  }
  int32_t end = min(len, start + tps);  // lowered to the new token's position when fused
  const int32_t n_pages = (end - 1) / bt - first_page + 1;  // <= max_pages

  int bad = 0;
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int32_t i = tid + k * NT;
    if (i < n_pages) {
      const bool ok = pg[k] < static_cast<uint32_t>(P.L.max_blocks);
      s_pages[i] = ok ? pg[k] : 0xFFFFFFFFu;
      bad |= ok ? 0 : 1;
    }
  }
  const bool clean = __syncthreads_or(bad) == 0;
  decode_state<D, G, Q8> S;
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4_t f = qraw[h][j];
      S.qh[h][2 * j] = pack_half2(f.x, f.y);
      S.qh[h][2 * j + 1] = pack_half2(f.z, f.w);
    }
    float qsum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qsum += static_cast<float>(S.qh[h][j].x) + static_cast<float>(S.qh[h][j].y);
    }
    S.kbias[h] = -1152.0f * qsum;
    if constexpr (MQK) {  // MFMA operand of head set h / 4: head h % 4 == lane % 4 (zero past G)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (h % 4 == 0) S.qm[h / 4][m] = half4_t{0, 0, 0, 0};
        if (h % 4 == (lane & 3)) {
          S.qm[h / 4][m] = half4_t{S.qh[h][2 * m].x, S.qh[h][2 * m].y, S.qh[h][2 * m + 1].x,
                                   S.qh[h][2 * m + 1].y};
        }
      }
      if (h % 4 == 0) S.kb[h / 4] = 0.0f;
      if (h % 4 == (lane & 3)) S.kb[h / 4] = S.kbias[h];
    }
    S.m[h] = -INFINITY;
    S.l[h] = 0.0f;
    if constexpr (Q8) S.vw[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) S.acc[h][i] = 0.0f;
  }

  const uint8_t *k_base = P.k_pool + static_cast<uint64_t>(P.layer) * P.L.layer_bytes +
                          static_cast<uint64_t>(kvh) * P.L.region_bytes;
  const uint8_t *v_base = P.v_pool + static_cast<uint64_t>(P.layer) * P.L.layer_bytes +
                          static_cast<uint64_t>(kvh) * P.L.region_bytes;
  const uint64_t page_bytes = P.L.page_bytes;
  // per-lane offsets of the UNIFORM path: row `grp` of the wave's rows
  const uint32_t lane_off =
      static_cast<uint32_t>(grp) * (Q8 ? D : 2 * D) + static_cast<uint32_t>(lane_in_row) * 16u;
  const uint32_t lane_sc_off =
      static_cast<uint32_t>(grp) * (D / 16) + static_cast<uint32_t>(lane_in_row / 2) * 2u;
  // MPV V words: the lane's 4 dims (mpv_dim) for the 4 tokens of its block
  [[maybe_unused]] const uint32_t lane_off_v =
      static_cast<uint32_t>(grp & ~3) * ROWB +
      static_cast<uint32_t>(mpv_dim<D, Q8>(lane_in_row, lane & 3)) * (Q8 ? 1u : 2u);
  auto load_v_quad = [&](const uint8_t *region, int32_t row0, row_regs<D, Q8> &r) {
    if constexpr (MPV) {
      const uint8_t *u = region + static_cast<uint32_t>(row0) * ROWB + lane_off_v;
      if constexpr (Q8) {
        r.a = uint4_t{load4_stream(u), load4_stream(u + D), load4_stream(u + 2 * D),
                      load4_stream(u + 3 * D)};
        const uint8_t *sc = region + static_cast<uint32_t>(bt) * D + static_cast<uint32_t>(row0) * (D / 16);
        r.d = load2_stream(sc + lane_sc_off);
      } else {
        const uint2_t t0 = load8_stream(u), t1 = load8_stream(u + ROWB);
        const uint2_t t2 = load8_stream(u + 2 * ROWB), t3 = load8_stream(u + 3 * ROWB);
        r.a = uint4_t{t0.x, t0.y, t1.x, t1.y};
        r.b = uint4_t{t2.x, t2.y, t3.x, t3.y};
      }
    }
  };

  // Fused append: the workgroup whose split holds position len - 1 stores
  // the new token and attends to it from registers after the memory tiles
  // (so nothing reads it back); the memory path ends before it.
  [[maybe_unused]] tile_regs<D, Q8> TN;
  bool has_new = false;
  bool new_ok = false;
  if (P.new_k != nullptr && len - 1 >= start && len - 1 < end) {  // uniform
    const int32_t p = len - 1;
    has_new = true;
    end = p;
    const uint32_t page = s_pages[p / bt - first_page];
    new_ok = page != 0xFFFFFFFFu;
    const uint64_t row = (static_cast<uint64_t>(seq) * P.L.n_head_kv + kvh) * D;
    new_row_regs<D, Q8>(P.new_k + row, lane_in_row, block_partner, TN.k0);
    new_row_regs<D, Q8>(P.new_v + row, lane_in_row, block_partner, TN.v0);
    if (new_ok && grp == 0) {
      const uint64_t region = static_cast<uint64_t>(P.layer) * P.L.layer_bytes +
                              static_cast<uint64_t>(kvh) * P.L.region_bytes +
                              static_cast<uint64_t>(page) * page_bytes;
      const int32_t off = p % bt;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        uint8_t *reg = (kv == 0 ? P.k_wr : P.v_wr) + region;
        const row_regs<D, Q8> &r = kv == 0 ? TN.k0 : TN.v0;
        if constexpr (!Q8) {
          uint8_t *dst = reg + static_cast<uint64_t>(off) * D * 2u + lane_in_row * 16u;
          store16(dst, r.a);
          store16(dst + D, r.b);
        } else {
          store16(reg + static_cast<uint64_t>(off) * D + lane_in_row * 16u, r.a);
          if ((lane_in_row & 1) == 0) {
            reinterpret_cast<uint16_t *>(reg + static_cast<uint64_t>(bt) * D)
                [static_cast<uint64_t>(off) * (D / 32) + lane_in_row / 2] =
                    static_cast<uint16_t>(r.d);
          }
        }
      }
    }
    // (after the store, which writes the row layout) V in the block
    // layout: token 0 of the quad only
    if constexpr (MPV && Q8) {
      const uint32_t wj[4] = {TN.v0.a.x, TN.v0.a.y, TN.v0.a.z, TN.v0.a.w};
      uint32_t w = wj[0];
#pragma unroll
      for (int k = 1; k < 4; ++k) w = (lane & 3) == k ? wj[k] : w;
      TN.v0.a = uint4_t{grp < 4 ? w : 0u, 0u, 0u, 0u};
    } else if constexpr (MPV) {  // f16: the two words of the lane's 4 dims
      const uint32_t wj[8] = {TN.v0.a.x, TN.v0.a.y, TN.v0.a.z, TN.v0.a.w,
                              TN.v0.b.x, TN.v0.b.y, TN.v0.b.z, TN.v0.b.w};
      uint32_t w0 = wj[0], w1 = wj[1];
#pragma unroll
      for (int k = 1; k < 4; ++k) {
        w0 = (lane & 3) == k ? wj[2 * k] : w0;
        w1 = (lane & 3) == k ? wj[2 * k + 1] : w1;
      }
      TN.v0.a = uint4_t{grp < 4 ? w0 : 0u, grp < 4 ? w1 : 0u, 0u, 0u};
      TN.v0.b = uint4_t{0u, 0u, 0u, 0u};
    }
    TN.k1 = TN.k0;
    TN.v1 = TN.v0;
  }

  // Loads the tile at `tbase` (rows past `end` and rows on invalid pages
  // read a valid clamped address and are reported in ok0/ok1).
  auto load_tile = [&](int32_t tbase, tile_regs<D, Q8> &T, bool &ok0, bool &ok1) {
    if constexpr (UNIFORM) {
      const int32_t ta = tbase;        // first token of half 0 (multiple of NGW)
      const int32_t tb = tbase + NGW;  // first token of half 1
      const bool hb = tb < end;
      // page index and row of both halves (uniform): shift and mask for
      // power-of-two pages, else a division
      int32_t ia, ib, rowa, rowb;
      if (P.bt_shift >= 0) {
        ia = ta >> P.bt_shift;
        ib = tb >> P.bt_shift;
        rowa = ta & (bt - 1);
        rowb = tb & (bt - 1);
      } else {
        ia = ta / bt;
        ib = tb / bt;
        rowa = ta - ia * bt;
        rowb = tb - ib * bt;
      }
      const uint32_t pa = __builtin_amdgcn_readfirstlane(s_pages[ia - first_page]);
      const uint32_t pb = hb ? __builtin_amdgcn_readfirstlane(s_pages[ib - first_page]) : pa;
      const bool va = pa != 0xFFFFFFFFu;
      const bool vb = pb != 0xFFFFFFFFu && hb;
      rowb = hb ? rowb : rowa;
      ok0 = va && ta + grp < end;
      ok1 = vb && tb + grp < end;
      const uint64_t ra = static_cast<uint64_t>(va ? pa : 0u) * page_bytes;
      const uint64_t rb = static_cast<uint64_t>(pb != 0xFFFFFFFFu ? pb : 0u) * page_bytes;
      load_row_uniform<D, Q8>(k_base + ra, rowa, lane_off, lane_sc_off, bt, T.k0);
      load_row_uniform<D, Q8>(k_base + rb, rowb, lane_off, lane_sc_off, bt, T.k1);
      if constexpr (MPV) {
        load_v_quad(v_base + ra, rowa, T.v0);
        load_v_quad(v_base + rb, rowb, T.v1);
      } else {
        load_row_uniform<D, Q8>(v_base + ra, rowa, lane_off, lane_sc_off, bt, T.v0);
        load_row_uniform<D, Q8>(v_base + rb, rowb, lane_off, lane_sc_off, bt, T.v1);
      }
    } else {
      const int32_t t0r = tbase + grp;
      const int32_t t1r = tbase + grp + NGW;
      const int32_t t0 = t0r < end ? t0r : start;
      const int32_t t1 = t1r < end ? t1r : start;
      const uint32_t p0 = s_pages[t0 / bt - first_page];
      const uint32_t p1 = s_pages[t1 / bt - first_page];
      ok0 = t0r < end && p0 != 0xFFFFFFFFu;
      ok1 = t1r < end && p1 != 0xFFFFFFFFu;
      const uint64_t r0 = static_cast<uint64_t>(p0 != 0xFFFFFFFFu ? p0 : 0u) * page_bytes;
      const uint64_t r1 = static_cast<uint64_t>(p1 != 0xFFFFFFFFu ? p1 : 0u) * page_bytes;
      load_row<D, Q8>(k_base + r0, t0 % bt, lane_in_row, bt, T.k0);
      load_row<D, Q8>(k_base + r1, t1 % bt, lane_in_row, bt, T.k1);
      load_row<D, Q8>(v_base + r0, t0 % bt, lane_in_row, bt, T.v0);
      load_row<D, Q8>(v_base + r1, t1 % bt, lane_in_row, bt, T.v1);
    }
  };

  // Full tiles of a split whose pages are all valid need no masks: they run
  // unmasked through two register sets used alternately by code position
  // (A, B, A, ...), so the next tile's loads stay in flight while the
  // current one is consumed.  (Rotating one set into another with moves
  // would force a wait for the in-flight loads.)  The split's partial last
  // tile, and every tile of a split with an invalid page, run masked after.
  const int32_t n_full = clean ? (end - start) / TT : 0;
  int32_t base = start;
  if (n_full > 0) {
    // Loads are unconditional (a load past the last full tile re-reads the
    // last full tile and is discarded): no branch around them, so the
    // compiler's wait counters keep NB - 1 tiles in flight across each
    // consume.  Register set j is only ever touched at unrolled position j.
    const int32_t last_full = start + (n_full - 1) * TT;
    tile_regs<D, Q8> R[NB];
    bool u0, u1;
#pragma unroll
    for (int j = 0; j + 1 < NB; ++j) {
      const int32_t t = start + j * TT;
      load_tile(t <= last_full ? t : last_full, R[j], u0, u1);
    }
    const int32_t n_groups = n_full / NB;
    for (int32_t i = 0; i < n_groups; ++i) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int32_t t = base + (NB - 1) * TT;
        load_tile(t <= last_full ? t : last_full, R[(j + NB - 1) % NB], u0, u1);
        consume_any<D, G, Q8, false, MQK, MPV>(S, R[j], true, true, P.c);
        base += TT;
      }
    }
    // the remaining n_full % NB tiles are already loaded into R[0..]
    const int32_t rem = n_full - n_groups * NB;
#pragma unroll
    for (int j = 0; j + 1 < NB; ++j) {
      if (j < rem) {
        consume_any<D, G, Q8, false, MQK, MPV>(S, R[j], true, true, P.c);
        base += TT;
      }
    }
  }
  for (; base < end; base += TT) {
    tile_regs<D, Q8> T;
    bool o0, o1;
    load_tile(base, T, o0, o1);
    consume_any<D, G, Q8, true, MQK, MPV>(S, T, o0, o1, P.c);
  }
  if (has_new) consume_any<D, G, Q8, true, MQK, MPV>(S, TN, new_ok && grp == 0, false, P.c);

  if constexpr (MPV) {
    // Lane (j, chunk, q) holds, for head set hs, head 4 hs + j's 16 dims of
    // its chunk over the tokens of its quad q: acc[hs][4 s + i] is dim 4 i + s
    // of the chunk.  Merge over the quad bits q (lane bits from 2 +
    // log2(LPT)) as the general path merges its token groups: rescale to the
    // common max, sum l, and halve the four 4-dim output chunks per exchange.
    constexpr int NHS = (G + 3) / 4;
    constexpr int RQ = __builtin_ctz(NGW / 4);
    constexpr int RS = RQ < 2 ? RQ : 2;
    constexpr int HELD = 16 >> RS;
    const int32_t quad = lane / (4 * LPT);
    int first_chunk = 0;
#pragma unroll
    for (int r = 0; r < RS; ++r) first_chunk += ((quad >> r) & 1) * (4 >> (r + 1));
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      const int32_t head = 4 * hs + (lane & 3);
      float M = S.m[hs];
#pragma unroll
      for (int r = 0; r < RQ; ++r) M = fmaxf(M, wave_shfl_xor(M, (4 * LPT) << r));
      const float ms = M == -INFINITY ? 0.0f : M;
      const float f = fast_exp2(S.m[hs] - ms);  // 0 for a lane that saw no token
      float l = S.l[hs] * f;
      float v[16];  // v[4 i + s]: dim 4 i + s, i.e. output chunk i in order
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int sd = 0; sd < 4; ++sd) {
          const float a =
              Q8 ? fmaf(-1152.0f, S.vw[hs], S.acc[hs][4 * sd + i]) : S.acc[hs][4 * sd + i];
          v[4 * i + sd] = a * f;
        }
      }
#pragma unroll
      for (int r = 0; r < RQ; ++r) l += wave_shfl_xor(l, (4 * LPT) << r);
#pragma unroll
      for (int r = 0; r < RS; ++r) {
        const int n = 16 >> r;
        const bool upper = (quad >> r) & 1;
#pragma unroll
        for (int k = 0; k < n / 2; ++k) {
          const float send = upper ? v[k] : v[k + n / 2];
          const float keep = upper ? v[k + n / 2] : v[k];
          v[k] = keep + wave_shfl_xor(send, (4 * LPT) << r);
        }
      }
#pragma unroll
      for (int r = RS; r < RQ; ++r) {
#pragma unroll
        for (int k = 0; k < HELD; ++k) v[k] += wave_shfl_xor(v[k], (4 * LPT) << r);
      }
      const bool writer = (quad >> RS) == 0 && head < G;
      const uint64_t row = static_cast<uint64_t>(seq) * P.L.n_head + kvh * G + head;
      if (P.direct_out != nullptr) {
        if (writer) {
          const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
          for (int cc = 0; cc < HELD / 4; ++cc) {
            *reinterpret_cast<float4_t *>(P.direct_out + row * D +
                                          mpv_dim<D, Q8>(lane_in_row, first_chunk + cc)) =
                float4_t{v[4 * cc] * inv, v[4 * cc + 1] * inv, v[4 * cc + 2] * inv,
                         v[4 * cc + 3] * inv};
          }
        }
        continue;
      }
      const uint64_t slot = slot_base + static_cast<uint64_t>(head) * slot_stride;
      if (writer) {
#pragma unroll
        for (int cc = 0; cc < HELD / 4; ++cc) {
          *reinterpret_cast<float4_t *>(P.part_acc + slot * D +
                                        mpv_dim<D, Q8>(lane_in_row, first_chunk + cc)) =
              float4_t{v[4 * cc], v[4 * cc + 1], v[4 * cc + 2], v[4 * cc + 3]};
        }
      }
      if (writer && lane_in_row == 0) {
        P.part_ml[slot * 2] = M;
        P.part_ml[slot * 2 + 1] = l;
      }
    }
    return;
  }
  if constexpr (Q8) {
    // acc holds sum w * (q + 1152): remove the bias term
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int i = 0; i < 16; ++i) S.acc[h][i] = fmaf(-1152.0f, S.vw[h], S.acc[h][i]);
    }
  }
  // Merge the wave's NGW token groups (lane bits >= log2(LPT)).  Every lane
  // first rescales its partial sums to the wave's max, so the rest is a
  // plain sum: l is summed across the groups, and acc is reduced by halving
  // exchanges (each round a lane sends the half of its float4 chunks its
  // partner keeps and adds the half it keeps), so after log2(NGW) rounds
  // each lane holds whole sums of NCH / NGW chunks instead of every lane
  // exchanging all G * 16 values each round.
  constexpr int NCH = G * 4;  // float4 chunks of acc: chunk c = (head c / 4, dims 4 * (c % 4))
  constexpr int R = __builtin_ctz(NGW);
  constexpr int RS = R < __builtin_ctz(NCH) ? R : __builtin_ctz(NCH);  // halving rounds
  float M[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    M[h] = S.m[h];
#pragma unroll
    for (int r = 0; r < R; ++r) M[h] = fmaxf(M[h], wave_shfl_xor(M[h], grp_mask(r)));
    const float ms = M[h] == -INFINITY ? 0.0f : M[h];
    const float f = fast_exp2(S.m[h] - ms);  // 0 for a lane that saw no token
    S.l[h] *= f;
#pragma unroll
    for (int i = 0; i < 16; ++i) S.acc[h][i] *= f;
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int r = 0; r < R; ++r) S.l[h] += wave_shfl_xor(S.l[h], grp_mask(r));
  }
  float (&v)[NCH * 4] = reinterpret_cast<float (&)[NCH * 4]>(S.acc);
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int n = (NCH >> r) * 4;  // floats held before this round
    const bool upper = (grp >> r) & 1;
#pragma unroll
    for (int k = 0; k < n / 2; ++k) {
      const float send = upper ? v[k] : v[k + n / 2];
      const float keep = upper ? v[k + n / 2] : v[k];
      v[k] = keep + wave_shfl_xor(send, grp_mask(r));
    }
  }
  constexpr int HELD = (NCH >> RS) * 4;  // floats held: chunks first_chunk .. + HELD / 4
#pragma unroll
  for (int r = RS; r < R; ++r) {  // more groups than chunks: sum what is held
#pragma unroll
    for (int k = 0; k < HELD; ++k) v[k] += wave_shfl_xor(v[k], grp_mask(r));
  }
  // the chunk index a lane holds: bit r of grp picks the upper half in round r
  int first_chunk = 0;
#pragma unroll
  for (int r = 0; r < RS; ++r) first_chunk += ((grp >> r) & 1) * (NCH >> (r + 1));
  const bool writer = (grp >> RS) == 0;  // one lane group per chunk after the sum rounds
  if (P.direct_out != nullptr) {  // the only split: o = acc / l
    if (writer) {
#pragma unroll
      for (int c = 0; c < HELD / 4; ++c) {
        const int ch = first_chunk + c;
        const int h = ch / 4;
        float l = S.l[0];
#pragma unroll
        for (int hh = 1; hh < G; ++hh) l = h == hh ? S.l[hh] : l;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *op = P.direct_out + (static_cast<uint64_t>(seq) * P.L.n_head + kvh * G + h) * D;
        *reinterpret_cast<float4_t *>(op + lane_dim<D, Q8>(lane_in_row, 4 * (ch % 4))) =
            float4_t{v[4 * c] * inv, v[4 * c + 1] * inv, v[4 * c + 2] * inv, v[4 * c + 3] * inv};
      }
    }
    return;
  }
  if (writer) {
#pragma unroll
    for (int c = 0; c < HELD / 4; ++c) {
      const int ch = first_chunk + c;
      const uint64_t slot = slot_base + static_cast<uint64_t>(ch / 4) * slot_stride;
      *reinterpret_cast<float4_t *>(P.part_acc + slot * D + lane_dim<D, Q8>(lane_in_row, 4 * (ch % 4))) =
          float4_t{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const uint64_t slot = slot_base + static_cast<uint64_t>(h) * slot_stride;
      P.part_ml[slot * 2] = M[h];
      P.part_ml[slot * 2 + 1] = S.l[h];
    }
  }
}

// Merging the splits inside the decode kernel instead (the last workgroup
// of a sequence, found by a device-scope completion count, merges) was
// measured slower at every decode shape on MI355X, 6.16 vs 6.38 TB/s at
// Llama-3-8B and 47 vs 37 us per Llama-3.2-1B layer even with one release
// per workgroup: the L2 writeback and invalidate that make partials
// written on one XCD visible on another cost more than this launch.
//
// Merges the split partials of one (sequence, head): o = sum_s 2^{m_s-M} acc_s
// / sum_s 2^{m_s-M} l_s (m in the log2 domain, scale folded in).
template <int D, int CH, bool BAL>
__global__ __launch_bounds__(D) void combine_kernel(const float *__restrict__ part_acc,
                                                     const float *__restrict__ part_ml,
                                                     const int32_t *__restrict__ kv_lens,
                                                     int32_t n_head, int32_t max_splits,
                                                     int32_t tokens_per_split,
                                                     float *__restrict__ out, int32_t n_seq,
                                                     int32_t host_tiles, int32_t tile) {
  const int32_t row = blockIdx.x;  // seq * n_head + head
  const int32_t seq = row / n_head;
  const int32_t d = threadIdx.x;
  // split s of this row is workspace row base + s * stride
  int32_t n;
  uint64_t base;
  [[maybe_unused]] uint64_t stride = 1u;
  if constexpr (BAL) {
    int32_t len_i, s_i, excl_i, tb;
    balanced_splits(kv_lens, n_seq, n_seq * max_splits, host_tiles, tile, d % k_wave, len_i, s_i,
                    excl_i, tb);
    // lengths past max_kv_len (outside the contract) could plan more splits
    // than the grid ran: read only slots the grid has
    const int32_t cap = n_seq * max_splits;
    const int32_t first = __builtin_amdgcn_readlane(excl_i, seq);
    n = __builtin_amdgcn_readlane(s_i, seq);
    n = first >= cap ? 0 : min(n, cap - first);
    base = static_cast<uint64_t>(first) * n_head + row % n_head;
    stride = static_cast<uint64_t>(n_head);
  } else {
    const int32_t len = kv_lens[seq];
    n = len > 0 ? min(max_splits, (len + tokens_per_split - 1) / tokens_per_split) : 0;
    base = static_cast<uint64_t>(row) * max_splits;
  }
  const float *ml = part_ml + base * 2;
  const float *pa = part_acc + base * D + d;
  // chunks of CH splits: every load of a chunk is issued before any is
  // used (one round trip for up to CH splits), with an online max across
  // chunks.  CH is 16 when a sequence has at most 16 splits, else 64
  // (measured: 16 is 3.5% faster at 15 splits, 64 is 4.7% faster at 33).
  // Issuing the first chunk's loads before the length arrives (bounded by
  // max_splits, or at clamped slots) measured slower: 176 and 159 vs 183
  // GB/s at Qwen3-0.6B, since the slots past the split count cost more than
  // the length's round trip saves.

  float mx = -INFINITY, l = 0.0f, a = 0.0f;
  for (int32_t s0 = 0; s0 < n; s0 += CH) {
    float mv[CH], lv[CH], av[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const bool in = s0 + u < n;
      const uint64_t k = BAL ? (s0 + u) * stride : static_cast<uint64_t>(s0 + u);
      mv[u] = in ? ml[2 * k] : -INFINITY;
      lv[u] = in ? ml[2 * k + 1] : 0.0f;
      av[u] = in ? pa[k * D] : 0.0f;
    }
    float cm = mv[0];
#pragma unroll
    for (int u = 1; u < CH; ++u) cm = fmaxf(cm, mv[u]);
    const float mn = fmaxf(mx, cm);
    const float ms = mn == -INFINITY ? 0.0f : mn;
    const float r = fast_exp2(mx - ms);  // 0 on the first chunk
    l *= r;
    a *= r;
    float lc[2] = {0.0f, 0.0f}, ac[2] = {0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const float f = fast_exp2(mv[u] - ms);  // 0 for splits past n
      lc[u & 1] = fmaf(lv[u], f, lc[u & 1]);
      ac[u & 1] = fmaf(av[u], f, ac[u & 1]);
    }
    l += lc[0] + lc[1];
    a += ac[0] + ac[1];
    mx = mn;
  }
  out[static_cast<uint64_t>(row) * D + d] = l > 0.0f ? a / l : 0.0f;
}

struct decode_plan {
  int32_t tokens_per_split = 0;
  int32_t max_splits = 0;
  uint64_t workspace_bytes = 0;
};

// Compute units of the current device, cached per device id.  Racing first
// calls store the same value, so relaxed atomics are enough.
int32_t device_cu_count() {
  static std::atomic<int32_t> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int32_t cus = cached[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        c <= 0) {
      c = 256;
    }
    cus = c;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// This is the host plan: the fixed split size, and the bound on the
// balanced plan the kernels derive on the device for 2 to 64 sequences
// (balanced_splits).
//
// Split sizing: about one workgroup per CU (a workgroup is 8 waves, which is
// what one CU holds at this kernel's register budget; more, shorter splits
// measured slower because every split pays its page-list load and merge),
// each split a whole number of wave tiles with its page list inside the LDS
// cache.
decode_plan plan_decode(const pool_layout &L, int32_t n_seq, int32_t max_kv_len) {
  decode_plan p;
  const int32_t lpt = L.head_dim / 16;
  const int32_t tile = 2 * (k_wave / lpt);
  const int32_t wpb = waves_per_block(L.n_head_kv);
  const int32_t units = n_seq * (L.n_head_kv / wpb);
  const int32_t target = device_cu_count();
  const int32_t tiles = (max_kv_len + tile - 1) / tile;
  int32_t splits = (target + units - 1) / units;
  splits = splits < 1 ? 1 : (splits > tiles ? tiles : splits);
  int32_t tps = ((max_kv_len + splits - 1) / splits + tile - 1) / tile * tile;
  const int32_t max_tps = ((k_max_split_pages - 2) * L.block_tokens) / tile * tile;
  if (tps > max_tps) tps = max_tps;
  if (tps < tile) tps = tile;
  p.tokens_per_split = tps;
  p.max_splits = (max_kv_len + tps - 1) / tps;
  p.workspace_bytes = static_cast<uint64_t>(n_seq) * L.n_head * p.max_splits *
                      static_cast<uint64_t>(L.head_dim + 2) * sizeof(float);
  return p;
}

template <int D, int G, bool Q8, int WPB>
void launch_decode_wpb(const decode_params &P, dim3 grid, hipStream_t st) {
  constexpr int NGW = k_wave / (D / 16);
  if (P.L.block_tokens % NGW == 0) {
    // MFMA scores and P.V (MPV) up to head_dim 256, any group size
    hipLaunchKernelGGL((decode_kernel<D, G, Q8, true, WPB, k_decode_nb, D <= 256, D <= 256>),
                       grid, dim3(WPB * k_wave), 0, st, P);
  } else {
    hipLaunchKernelGGL((decode_kernel<D, G, Q8, false, WPB, k_decode_nb, Q8 && D <= 256, false>),
                       grid, dim3(WPB * k_wave), 0, st, P);
  }
}

template <int D, int G, bool Q8>
void launch_decode(const decode_params &P, dim3 grid, hipStream_t st) {
  switch (waves_per_block(P.L.n_head_kv)) {
    case 8: launch_decode_wpb<D, G, Q8, 8>(P, grid, st); break;
    case 4: launch_decode_wpb<D, G, Q8, 4>(P, grid, st); break;
    case 2: launch_decode_wpb<D, G, Q8, 2>(P, grid, st); break;
    default: launch_decode_wpb<D, G, Q8, 1>(P, grid, st); break;
  }
}

template <int D, bool Q8>
bool dispatch_group(int32_t group, const decode_params &P, dim3 grid, hipStream_t st) {
  switch (group) {
    case 1: launch_decode<D, 1, Q8>(P, grid, st); return true;
    case 2: launch_decode<D, 2, Q8>(P, grid, st); return true;
    case 4: launch_decode<D, 4, Q8>(P, grid, st); return true;
    case 8: launch_decode<D, 8, Q8>(P, grid, st); return true;
    default: return false;
  }
}

template <bool Q8>
bool dispatch_dim(int32_t head_dim, int32_t group, const decode_params &P, dim3 grid,
                  hipStream_t st) {
  switch (head_dim) {
    case 64: return dispatch_group<64, Q8>(group, P, grid, st);
    case 128: return dispatch_group<128, Q8>(group, P, grid, st);
    case 256: return dispatch_group<256, Q8>(group, P, grid, st);
    case 512: return dispatch_group<512, Q8>(group, P, grid, st);
    default: return false;
  }
}

bool dispatch_decode(const pool_layout &L, const decode_params &P, dim3 grid, hipStream_t st) {
  const int32_t group = L.n_head / L.n_head_kv;
  return L.kv_type == EMELK_KV_Q8_0 ? dispatch_dim<true>(L.head_dim, group, P, grid, st)
                                    : dispatch_dim<false>(L.head_dim, group, P, grid, st);
}

template <int D, int CH>
void launch_combine_d(dim3 grid, hipStream_t st, const decode_params &P, const int32_t *kv_lens,
                      int32_t n_head, int32_t max_splits, int32_t tps, float *out, int32_t n_seq,
                      int32_t tile) {
  if (P.balanced) {
    hipLaunchKernelGGL((combine_kernel<D, CH, true>), grid, dim3(D), 0, st, P.part_acc, P.part_ml,
                       kv_lens, n_head, max_splits, tps, out, n_seq, P.host_tiles, tile);
  } else {
    hipLaunchKernelGGL((combine_kernel<D, CH, false>), grid, dim3(D), 0, st, P.part_acc, P.part_ml,
                       kv_lens, n_head, max_splits, tps, out, n_seq, P.host_tiles, tile);
  }
}

template <int CH>
void launch_combine_ch(int32_t head_dim, dim3 grid, hipStream_t st, const decode_params &P,
                       const int32_t *kv_lens, int32_t n_head, int32_t max_splits, int32_t tps,
                       float *out, int32_t n_seq, int32_t tile) {
  switch (head_dim) {
    case 64: launch_combine_d<64, CH>(grid, st, P, kv_lens, n_head, max_splits, tps, out, n_seq, tile); break;
    case 128: launch_combine_d<128, CH>(grid, st, P, kv_lens, n_head, max_splits, tps, out, n_seq, tile); break;
    case 256: launch_combine_d<256, CH>(grid, st, P, kv_lens, n_head, max_splits, tps, out, n_seq, tile); break;
    default: launch_combine_d<512, CH>(grid, st, P, kv_lens, n_head, max_splits, tps, out, n_seq, tile); break;
  }
}

}  // namespace

// Chunked prefill on q8_0 pools, row by row as run_prefill does
// (text/generator/detail.hpp:4297-4372): row r of sequence s is a decode of
// q_start[s] + r + 1 tokens through s's block-table row, one split per row,
// written straight to out (no workspace).  The context of a row must fit
// one split's page list (k_max_split_pages - 2 pages).
emel_error_type decode_rows(const pool_layout &L, const void *k_pool, const void *v_pool,
                            int32_t layer, const float *q, float *out, int32_t n_seq, int32_t n_q,
                            const int32_t *q_start, const uint16_t *block_tables,
                            int32_t table_stride, float scale, hipStream_t st) {
  const int64_t n_rows = static_cast<int64_t>(n_seq) * n_q;
  if (n_rows > 65535) return EMELK_ERR_INVALID_REQUEST;
  const int32_t tile = 2 * (k_wave / (L.head_dim / 16));
  const int64_t bound = static_cast<int64_t>(table_stride) * L.block_tokens;  // longest row context
  const int64_t max_tps = static_cast<int64_t>(k_max_split_pages - 2) * L.block_tokens / tile * tile;
  const int64_t tps = (bound + tile - 1) / tile * tile;
  if (tps > max_tps) return EMELK_ERR_INVALID_REQUEST;
  decode_params P{};
  P.L = L;
  P.k_pool = static_cast<const uint8_t *>(k_pool);
  P.v_pool = static_cast<const uint8_t *>(v_pool);
  P.layer = layer;
  P.q = q;
  P.kv_lens = nullptr;
  P.tables = block_tables;
  P.table_stride = table_stride;
  P.c = scale * 1.4426950408889634f;
  P.tokens_per_split = static_cast<int32_t>(tps);
  P.max_splits = 1;
  P.part_acc = nullptr;
  P.part_ml = nullptr;
  P.new_k = nullptr;
  P.new_v = nullptr;
  P.k_wr = nullptr;
  P.v_wr = nullptr;
  P.direct_out = out;
  P.row_q_start = q_start;
  P.rows = n_q;
  P.balanced = 0;
  P.host_tiles = 0;
  P.bt_shift = pow2_shift(L.block_tokens);
  const dim3 grid(1, L.n_head_kv / waves_per_block(L.n_head_kv), static_cast<uint32_t>(n_rows));
  if (!dispatch_decode(L, P, grid, st)) return EMELK_ERR_INVALID_REQUEST;
  return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
}

}  // namespace emelk

// The split count grows as the batch shrinks (about one workgroup per CU is
// the target), so n_seq * splits is not monotone in n_seq.  A workspace sized
// for (n_seq, max_kv_len) must serve every call with fewer sequences or
// shorter contexts, which is what an executor sized for its largest step
// relies on; the size returned is the maximum of the exact need over all
// n' <= n_seq, len' <= max_kv_len.  For a fixed n', splits(n', len') <=
// max(min(ceil(target / units'), tiles(len')), ceil(len' / max_tps)), which
// is nondecreasing in len', so the bound at len' = max_kv_len covers them.
extern "C" emel_error_type emelk_attn_decode_workspace_size(const emelk_kv_geometry *g,
                                                            int32_t n_seq, int32_t max_kv_len,
                                                            uint64_t *bytes_out) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || bytes_out == nullptr || n_seq <= 0 ||
      n_seq > 65535 || max_kv_len <= 0) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  const int32_t tile = 2 * (emelk::k_wave / (L.head_dim / 16));
  const int32_t wpb = emelk::waves_per_block(L.n_head_kv);
  const int32_t target = emelk::device_cu_count();
  const int64_t tiles = (static_cast<int64_t>(max_kv_len) + tile - 1) / tile;
  const int64_t max_tps = ((emelk::k_max_split_pages - 2) * L.block_tokens) / tile * tile;
  const int64_t clamp_splits = (max_kv_len + max_tps - 1) / max_tps;
  uint64_t worst = 0;
  for (int64_t n = 1; n <= n_seq; ++n) {
    const int64_t units = n * (L.n_head_kv / wpb);
    int64_t splits = (target + units - 1) / units;
    if (splits > tiles) splits = tiles;
    if (splits < clamp_splits) splits = clamp_splits;
    if (static_cast<uint64_t>(n * splits) > worst) worst = static_cast<uint64_t>(n * splits);
  }
  *bytes_out = worst * L.n_head * static_cast<uint64_t>(L.head_dim + 2) * sizeof(float);
  return EMELK_ERR_NONE;
}

extern "C" emel_error_type emelk_attn_decode_plan(const emelk_kv_geometry *g, int32_t n_seq,
                                                  int32_t max_kv_len, int32_t *tokens_per_split,
                                                  int32_t *n_splits, uint64_t *bytes_out) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || n_seq <= 0 || n_seq > 65535 ||
      max_kv_len <= 0) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  const emelk::decode_plan p = emelk::plan_decode(L, n_seq, max_kv_len);
  if (tokens_per_split != nullptr) *tokens_per_split = p.tokens_per_split;
  if (n_splits != nullptr) *n_splits = p.max_splits;
  if (bytes_out != nullptr) *bytes_out = p.workspace_bytes;
  return EMELK_ERR_NONE;
}

namespace {

emel_error_type decode_impl(const emelk_kv_geometry *g, const void *k_pool, const void *v_pool,
                            int32_t layer, const float *q, float *out, int32_t n_seq,
                            const int32_t *kv_lens, int32_t max_kv_len,
                            const uint16_t *block_tables, int32_t table_stride, float scale,
                            void *workspace, uint64_t workspace_bytes, void *stream,
                            const float *new_k, const float *new_v) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || k_pool == nullptr || v_pool == nullptr ||
      q == nullptr || out == nullptr || kv_lens == nullptr || workspace == nullptr || layer < 0 ||
      layer >= L.n_layer || n_seq <= 0 || n_seq > 65535 || max_kv_len <= 0 ||
      table_stride <= 0 || !(scale > 0.0f) || !std::isfinite(scale)) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  const emelk::decode_plan plan = emelk::plan_decode(L, n_seq, max_kv_len);
  if (workspace_bytes < plan.workspace_bytes) return EMELK_ERR_INVALID_REQUEST;
  emelk::decode_params P;
  P.L = L;
  P.k_pool = static_cast<const uint8_t *>(k_pool);
  P.v_pool = static_cast<const uint8_t *>(v_pool);
  P.layer = layer;
  P.q = q;
  P.kv_lens = kv_lens;
  P.tables = block_tables;
  P.table_stride = table_stride;
  P.c = scale * 1.4426950408889634f;
  P.tokens_per_split = plan.tokens_per_split;
  P.max_splits = plan.max_splits;
  P.new_k = new_k;
  P.new_v = new_v;
  // a single split per sequence needs no merge: the decode kernel writes out
  P.direct_out = plan.max_splits == 1 ? out : nullptr;
  P.row_q_start = nullptr;
  P.rows = 1;
  // balanced splits for a ragged batch: every split about the same size
  const int32_t tile = 2 * (emelk::k_wave / (L.head_dim / 16));
  P.balanced = plan.max_splits > 1 && n_seq > 1 && n_seq <= emelk::k_wave ? 1 : 0;
  P.host_tiles = plan.tokens_per_split / tile;
  P.bt_shift = emelk::pow2_shift(L.block_tokens);
  P.k_wr = static_cast<uint8_t *>(const_cast<void *>(k_pool));
  P.v_wr = static_cast<uint8_t *>(const_cast<void *>(v_pool));
  const uint64_t acc_floats = static_cast<uint64_t>(n_seq) * L.n_head * plan.max_splits * L.head_dim;
  P.part_acc = static_cast<float *>(workspace);
  P.part_ml = P.part_acc + acc_floats;
  const dim3 grid(plan.max_splits, L.n_head_kv / emelk::waves_per_block(L.n_head_kv), n_seq);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!emelk::dispatch_decode(L, P, grid, st)) return EMELK_ERR_INVALID_REQUEST;
  if (P.direct_out != nullptr) return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
  const dim3 cgrid(n_seq * L.n_head);
  if (plan.max_splits > 16) {
    emelk::launch_combine_ch<64>(L.head_dim, cgrid, st, P, kv_lens, L.n_head, plan.max_splits,
                                 plan.tokens_per_split, out, n_seq, tile);
  } else {
    emelk::launch_combine_ch<16>(L.head_dim, cgrid, st, P, kv_lens, L.n_head, plan.max_splits,
                                 plan.tokens_per_split, out, n_seq, tile);
  }
  return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
}

}  // namespace

extern "C" emel_error_type emelk_attn_decode(const emelk_kv_geometry *g, const void *k_pool,
                                             const void *v_pool, int32_t layer, const float *q,
                                             float *out, int32_t n_seq, const int32_t *kv_lens,
                                             int32_t max_kv_len, const uint16_t *block_tables,
                                             int32_t table_stride, float scale, void *workspace,
                                             uint64_t workspace_bytes, void *stream) {
  if (block_tables == nullptr) return EMELK_ERR_INVALID_REQUEST;
  return decode_impl(g, k_pool, v_pool, layer, q, out, n_seq, kv_lens, max_kv_len, block_tables,
                     table_stride, scale, workspace, workspace_bytes, stream, nullptr, nullptr);
}

extern "C" emel_error_type emelk_attn_decode_append(
    const emelk_kv_geometry *g, void *k_pool, void *v_pool, int32_t layer, const float *k_rows,
    const float *v_rows, const float *q, float *out, int32_t n_seq, const int32_t *kv_lens,
    int32_t max_kv_len, const uint16_t *block_tables, int32_t table_stride, float scale,
    void *workspace, uint64_t workspace_bytes, void *stream) {
  if (k_rows == nullptr || v_rows == nullptr || block_tables == nullptr) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  return decode_impl(g, k_pool, v_pool, layer, q, out, n_seq, kv_lens, max_kv_len, block_tables,
                     table_stride, scale, workspace, workspace_bytes, stream, k_rows, v_rows);
}

// Contiguous caches: sequence s holds its tokens in pages s * pages_per_seq
// onwards, in order, so no block table is read.  One page spanning the
// capacity (max_blocks = 1) makes the pools the flash route's head-major
// caches (text/generator/detail.hpp:3232-3292).
extern "C" emel_error_type emelk_attn_decode_contiguous(
    const emelk_kv_geometry *g, void *k_pool, void *v_pool, int32_t layer, const float *k_rows,
    const float *v_rows, const float *q, float *out, int32_t n_seq, const int32_t *kv_lens,
    int32_t max_kv_len, int32_t seq_stride_tokens, float scale, void *workspace,
    uint64_t workspace_bytes, void *stream) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || (k_rows == nullptr) != (v_rows == nullptr) ||
      n_seq <= 0 || n_seq > 65535 || seq_stride_tokens <= 0 ||
      seq_stride_tokens % L.block_tokens != 0 || max_kv_len > seq_stride_tokens) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  const int64_t pages_per_seq = seq_stride_tokens / L.block_tokens;
  if (pages_per_seq * n_seq > L.max_blocks) return EMELK_ERR_INVALID_REQUEST;
  return decode_impl(g, k_pool, v_pool, layer, q, out, n_seq, kv_lens, max_kv_len, nullptr,
                     static_cast<int32_t>(pages_per_seq), scale, workspace, workspace_bytes,
                     stream, k_rows, v_rows);
}

// ---- allocation-free variant -----------------------------------------------
// The split partials live in a file-scope device array instead of a caller
// workspace.  Each GPU the library runs on holds its own copy (sized
// EMELK_DECODE_STATIC_SCRATCH_BYTES) until the process ends.  In host code
// `scratch` names a host-side stand-in, never a device address: the address
// of this device's copy comes from hipGetSymbolAddress, looked up once per
// device with that device current, and only that address is handed to
// kernels.  Nothing in the partials must start at zero (every split a
// combine reads was written by this call's decode launch), so no clearing
// runs.  Calls that overlap on one GPU share the array and race.
namespace {

static __device__ __align__(256) uint8_t scratch[EMELK_DECODE_STATIC_SCRATCH_BYTES];

constexpr int k_max_devices = 64;
std::atomic<void *> scratch_ptr[k_max_devices];

// The copy of `scratch` on the device of `stream`, which must be the current
// device (the symbol lookup resolves on the current device); nullptr with
// *err set otherwise.  A null stream is the current device's.
void *device_scratch(void *stream, emel_error_type *err) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= k_max_devices) {
    *err = EMELK_ERR_BACKEND;
    return nullptr;
  }
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess) {
      *err = EMELK_ERR_BACKEND;
      return nullptr;
    }
    if (sdev != dev) {  // another GPU's stream: its kernels must not get this GPU's array
      *err = EMELK_ERR_INVALID_REQUEST;
      return nullptr;
    }
  }
  void *p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    // racing first calls on one device look up the same address
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      *err = EMELK_ERR_BACKEND;
      return nullptr;
    }
    scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace

extern "C" emel_error_type emelk_attn_decode_noalloc(
    const emelk_kv_geometry *g, void *k_pool, void *v_pool, int32_t layer, const float *k_rows,
    const float *v_rows, const float *q, float *out, int32_t n_seq, const int32_t *kv_lens,
    int32_t max_kv_len, const uint16_t *block_tables, int32_t table_stride, float scale,
    void *stream) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || n_seq <= 0 || n_seq > 65535 ||
      max_kv_len <= 0 || ((k_rows == nullptr) != (v_rows == nullptr))) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  // the exact need of this call, checked before the device is touched
  if (emelk::plan_decode(L, n_seq, max_kv_len).workspace_bytes > EMELK_DECODE_STATIC_SCRATCH_BYTES) {
    return EMELK_ERR_OUT_OF_MEMORY;
  }
  // decode_impl's remaining argument checks, also before the device is touched
  if (k_pool == nullptr || v_pool == nullptr || q == nullptr || out == nullptr ||
      kv_lens == nullptr || block_tables == nullptr || layer < 0 || layer >= L.n_layer ||
      table_stride <= 0 || !(scale > 0.0f) || !std::isfinite(scale)) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  emel_error_type err = EMELK_ERR_NONE;
  void *ws = device_scratch(stream, &err);
  if (ws == nullptr) return err;
  return decode_impl(g, k_pool, v_pool, layer, q, out, n_seq, kv_lens, max_kv_len, block_tables,
                     table_stride, scale, ws, EMELK_DECODE_STATIC_SCRATCH_BYTES, stream, k_rows,
                     v_rows);
}
