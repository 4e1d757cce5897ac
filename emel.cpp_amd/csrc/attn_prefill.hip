// Chunked-prefill attention on MFMA (gfx950 v_mfma_f32_32x32x16_f16).
//
// Replaces the reference's per-row chunked prefill (run_prefill's store +
// attend loop, text/generator/detail.hpp:4297-4372: row r of the chunk
// attends causally to logical positions [0, q_start + r]) with one flash
// attention pass per chunk.
//
// Workgroup = 8 waves = one KV head, G_WG query heads of its group and RB
// row blocks of 32 query rows (G_WG * RB = 8), so the eight waves share
// every K/V tile staged in LDS (256 flops per staged byte at D = 128).  A
// key tile is KT = 64 keys in two 32-key sub-tiles; per sub-tile each wave
// computes
//     S^T (32 keys x 32 rows)  = K (32 x D) . Q^T (D x 32)      D/16 MFMAs
// so a lane holds 16 of the 32 scores of ONE query row (the other 16 sit in
// the lane 32 apart): the row max and sum are in-lane plus one cross-half
// swap (v_permlane32_swap).  The fp32 score accumulator converted to fp16
// is directly the A operand of
//     O (32 rows x D) += P (32 x 32 keys) . V (32 x D)        2*D/32 MFMAs
// provided the keys of V are staged in LDS in the order the accumulator
// holds them (key_slot below), which the staging does while transposing V.
// Online softmax in fp32 (exp2 with the scale folded in, lazy rescale); Q
// is rounded to fp16 as round_q_for_nonflash does (detail.hpp:2898-2903)
// and P is fp16, as the reference's rounded probabilities are
// (detail.hpp:3146-3149).  K/V tiles are double-buffered in LDS: the next
// tile's global loads are issued before the current tile's MFMAs.  Keys on
// invalid pages are left out of the softmax, as in decode.
#include <hip/hip_runtime.h>

#include <cmath>

#include "device_common.hpp"
#include "emelk.h"
#include "decode_rows.hpp"
#include "pool_layout.hpp"

namespace emelk {
namespace {

using namespace emelk::dev;

constexpr int k_sub = 32;   // keys per MFMA sub-tile (one score accumulator)
constexpr float k_rescale = 8.0f;  // lazy-rescale threshold (log2 units)
constexpr int k_max_seq_pages = EMELK_MAX_BLOCKS_PER_SEQUENCE;  // LDS page list
// word 3 of a raw buffer resource (gfx9 family): 32-bit data format, no
// swizzle, offsets checked against num_records
constexpr int k_rsrc_word3 = 0x00020000;

typedef _Float16 half8_v __attribute__((ext_vector_type(8)));
typedef float float16_v __attribute__((ext_vector_type(16)));
typedef uint32_t uint2_v __attribute__((ext_vector_type(2)));

struct prefill_params {
  pool_layout L;
  const uint8_t *k_pool;
  const uint8_t *v_pool;
  int32_t layer;
  const float *q;  // [n_seq][n_q][n_head][D]
  float *out;      // same shape
  int32_t n_q;
  const int32_t *q_start;
  const uint16_t *tables;
  int32_t table_stride;
  float c;  // scale * log2(e)
  int32_t bt_shift;  // log2(block_tokens) when a power of two, else -1
};

// Register staging of one key tile.  f16 pools: K as 16-byte row chunks, V
// as 4 keys x 2 dims.  q8_0 pools: the same items at one byte per value plus
// each value block's fp16 scale (V words hold the int8 pair in the low and
// the scale in the high 16 bits); they become fp16 when written to LDS.
template <int KI, int VI, bool Q8>
struct prefill_stage {
  uint4_t rk[KI];
  uint32_t rv[VI][4];
};
template <int KI, int VI>
struct prefill_stage<KI, VI, true> {
  uint2_v rk[KI];
  uint32_t ks[KI];
  uint32_t rv[VI][4];
};

// q8_0 -> two fp16 planes for LDS whose sum is exactly q * d, so the MFMAs
// see the dequantized values of dequantize_row_q8_0 (kernel/detail.hpp:
// 679-690) without rounding: q is exact in fp16 (a byte under the exponent
// of 1024, biased by 1152); hi = fp16(q * d) and lo = fma(q, d, -hi), which
// is exact: q * d has at most 7 + 11 significant bits, hi holds the top 11,
// and the remainder is a multiple of d's ulp (>= 2^-24, an fp16 subnormal
// step) below 2^7 of them.  Two values per packed op.  Only |q * d| at or
// beyond 65520 (outside fp16) does not hold, since hi is then infinite.
// Returns (hi, lo).  K is staged as both planes: the scores stay exact, since
// a rounding of K moves a score by up to 2^-11 of sum |q k|, which the
// softmax amplifies past the 2e-3 bar on data with x20 outliers.  V is staged
// as both planes too, and P as an fp16 hi + lo pair: the P.V MFMAs take
// P_hi V_hi + P_hi V_lo + P_lo V_hi.  With one fp16 rounding of V (hi alone)
// and of P, the GPU's own rounding added to the reference route's rounding
// of its probabilities and went past the bar on x20-outlier data (1.04 of
// it on a seeded sweep); with both carried this far the GPU's distance to
// the reference is the reference's own (0.46 of the bar on the same cases).
__device__ __forceinline__ uint2_v q8_pair_to_f16x2(uint32_t bytes2, half2_t d2) {
  const uint32_t u = bytes2 ^ 0x8080u;
  const half2_t q = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) -
                    half2_t{1152, 1152};
  const half2_t h = q * d2;
  return uint2_v{as_u32(h), as_u32(__builtin_elementwise_fma(q, d2, -h))};
}

// Slot of key k (0..31) in the MFMA k-order of the score accumulator:
// accumulator register r of lane-half h holds key 8*(r/4) + 4*h + r%4; the
// P operand of k-step s uses registers 8s..8s+7, i.e. slot s*16 + 8*h + i
// holds key 16*s + 8*(i/4) + 4*h + i%4.
__device__ __forceinline__ int key_slot(int k) {
  const int s = k >> 4;
  const int rem = k & 15;
  const int i = ((rem >> 3) << 2) | (rem & 3);
  const int h = (rem >> 2) & 1;
  return s * 16 + h * 8 + i;
}

// Slot of key k (0..31) for the 16-row layout (v_mfma_f32_16x16x32_f16):
// the score accumulators of a lane group g = lane/16 hold keys 4g..4g+3 and
// 16+4g..16+4g+3 of its query row, which are P operand k-indices 8g..8g+7.
__device__ __forceinline__ int key_slot16(int k) {
  return 8 * ((k & 15) >> 2) + (k >= 16 ? 4 : 0) + (k & 3);
}

typedef float float4_v __attribute__((ext_vector_type(4)));

template <int D, int G_WG, int RB, int KT, bool Q8, bool M16 = false>
__global__ __launch_bounds__(G_WG * RB * k_wave) void prefill_kernel(prefill_params P) {
  constexpr int WAVES = G_WG * RB;
  constexpr int NT = WAVES * k_wave;
  constexpr int KSTEPS = D / 16;   // MFMA k-steps for S^T
  constexpr int DCH = D / 32;      // 32-wide dim chunks of O
  // M16: 16 query rows per wave on v_mfma_f32_16x16x32_f16 (head_dim 512,
  // whose 32-row O tile and Q^T operand do not fit one wave's registers)
  constexpr int ROWS = M16 ? 16 : 32;
  constexpr int KS16 = D / 32;     // M16: k-steps of 32 dims
  constexpr int OT16 = D / 16;     // M16: 16-column tiles of O
  constexpr int KROW = D + 8;      // padded LDS row (halves) of K
  constexpr int NS = KT / k_sub;   // score sub-tiles per key tile
  constexpr int VROW = KT + 8;     // padded LDS row (halves) of V^T
  // staging items per 32-key tile: K in 8-half chunks, V in (4 keys x 2 dims)
  constexpr int KITEMS = KT * D / 8;
  constexpr int VITEMS = (KT / 4) * (D / 2);
  constexpr int KI = (KITEMS + NT - 1) / NT;
  constexpr int VI = (VITEMS + NT - 1) / NT;
  constexpr uint32_t ROWB = Q8 ? D : 2 * D;  // bytes of one K/V row in a page
  constexpr uint32_t SROWB = D / 16;         // q8_0: bytes of one row's scales

  // q8_0: a hi and a lo plane of K (their sum is exact); V^T is one plane
  // of fp16(q * d) for both pool types
  constexpr int PL = Q8 ? 2 : 1;
  __shared__ half_t s_k[2][PL][KT][KROW];
  constexpr int VR = 2;  // V double buffer
  // q8_0: V^T as a hi and a lo plane as well (their sum is exact), so P.V
  // sees the dequantized values unrounded
  __shared__ half_t s_vt[VR][PL][D][VROW];
  __shared__ float s_row[WAVES][32];
  __shared__ uint16_t s_ptab[k_max_seq_pages];

  // Workgroup -> (query tile, head group, sequence).  Consecutive workgroup
  // ids are spread over the 8 XCDs; the mapping gives each XCD a contiguous
  // run of (head group, sequence) units with all their query tiles, so the
  // tiles that re-read one unit's K/V share that XCD's L2.
  const int n_qt = (P.n_q + RB * ROWS - 1) / (RB * ROWS);
  const int n_hg = P.L.n_head / G_WG;
  const int total_wg = gridDim.x;
  int lin = blockIdx.x;
  int qt, unit;
  const int run = total_wg >> 3;  // workgroups per XCD
  if (Q8 && (total_wg & 7) == 0 && run % n_qt == 0) {
    // q8_0: dispatch order k inside an XCD's run gives the run's units
    // with their longest (latest) query tiles first, so the CUs that finish
    // a short tile first take the longest of the rest (config-5 shape:
    // 615 vs 632 us; no change for f16, where it stays off)
    const int k = blockIdx.x >> 3;
    const int ux = run / n_qt;  // units per XCD
    unit = (blockIdx.x & 7) * ux + k % ux;
    qt = n_qt - 1 - k / ux;
  } else {
    if ((total_wg & 7) == 0) lin = (blockIdx.x >> 3) + run * (blockIdx.x & 7);
    qt = lin % n_qt;
    unit = lin / n_qt;
  }
  const int hg = unit % n_hg;
  const int seq = unit / n_hg;

  const int tid = threadIdx.x;
  const int wave = tid / k_wave;
  const int lane = tid % k_wave;
  const int h = lane / 32;
  const int l32 = lane % 32;
  const int group = P.L.n_head / P.L.n_head_kv;
  const int head0 = hg * G_WG;
  const int kvh = head0 / group;
  const int head = head0 + wave % G_WG;
  const int row0 = (qt * RB + wave / G_WG) * ROWS;
  const int c16 = lane % 16;  // M16: the lane's query row (and O column) in its block
  const int g16 = lane / 16;  // M16: lane group
  const int n_q = P.n_q;
  const int q0 = P.q_start[seq];
  // a negative q_start names no valid position: the sequence attends to
  // nothing (no tiles, no page lookups) and its rows are written as zeros
  const bool seq_ok = q0 >= 0;
  const int total = seq_ok ? q0 + n_q : 0;
  const int wg_row_end = min(n_q, (qt + 1) * RB * ROWS);
  const int key_end = seq_ok ? q0 + wg_row_end : 0;  // exclusive
  const int n_tiles = (key_end + KT - 1) / KT;
  const int my_row = row0 + (M16 ? c16 : l32);
  const bool row_ok = my_row < n_q;
  const int my_pos = q0 + my_row;
  const int wg_first_pos = q0 + qt * RB * ROWS;  // smallest query position in the WG

  // Q^T operand (B): lane holds query my_row, dims 16*kk + 8*h .. +7
  // (M16: dims 32*kk + 8*g16 .. +7).
  half8_v qop[M16 ? 1 : KSTEPS];
  half8_v qop16[M16 ? KS16 : 1];
  if constexpr (M16) {
    const float *qp = P.q + ((static_cast<uint64_t>(seq) * n_q + (row_ok ? my_row : 0)) *
                                 P.L.n_head + head) * D;
#pragma unroll
    for (int kk = 0; kk < KS16; ++kk) {
      const float4_t a = *reinterpret_cast<const float4_t *>(qp + 32 * kk + 8 * g16);
      const float4_t b = *reinterpret_cast<const float4_t *>(qp + 32 * kk + 8 * g16 + 4);
      half8_v v;
      v[0] = static_cast<half_t>(a.x); v[1] = static_cast<half_t>(a.y);
      v[2] = static_cast<half_t>(a.z); v[3] = static_cast<half_t>(a.w);
      v[4] = static_cast<half_t>(b.x); v[5] = static_cast<half_t>(b.y);
      v[6] = static_cast<half_t>(b.z); v[7] = static_cast<half_t>(b.w);
      if (!row_ok) v = half8_v{0, 0, 0, 0, 0, 0, 0, 0};
      qop16[kk] = v;
    }
  } else {
    const float *qp = P.q + ((static_cast<uint64_t>(seq) * n_q + (row_ok ? my_row : 0)) *
                                 P.L.n_head + head) * D;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const float4_t a = *reinterpret_cast<const float4_t *>(qp + 16 * kk + 8 * h);
      const float4_t b = *reinterpret_cast<const float4_t *>(qp + 16 * kk + 8 * h + 4);
      half8_v v;
      v[0] = static_cast<half_t>(a.x); v[1] = static_cast<half_t>(a.y);
      v[2] = static_cast<half_t>(a.z); v[3] = static_cast<half_t>(a.w);
      v[4] = static_cast<half_t>(b.x); v[5] = static_cast<half_t>(b.y);
      v[6] = static_cast<half_t>(b.z); v[7] = static_cast<half_t>(b.w);
      if (!row_ok) v = half8_v{0, 0, 0, 0, 0, 0, 0, 0};
      qop[kk] = v;
    }
  }

  float16_v o[M16 ? 1 : DCH];
  float4_v o16[M16 ? OT16 : 1];
#pragma unroll
  for (int c = 0; c < (M16 ? 1 : DCH); ++c) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[c][r] = 0.0f;
  }
#pragma unroll
  for (int c = 0; c < (M16 ? OT16 : 1); ++c) o16[c] = float4_v{0.0f, 0.0f, 0.0f, 0.0f};
  float m = -INFINITY;  // raw-score reference max of this lane's row
  float l = 0.0f;
  const float rescale_raw = k_rescale / P.c;

  const uint64_t layer_base = static_cast<uint64_t>(P.layer) * P.L.layer_bytes +
                              static_cast<uint64_t>(kvh) * P.L.region_bytes;
  const uint16_t *table = P.tables + static_cast<uint64_t>(seq) * P.table_stride;
  // LDS copy of the page list for every page the workgroup's tiles touch
  // (the last tile can reach past key_end); lookups beyond n_pt read as
  // invalid.  `clean` when every page the workgroup reads is valid (keys on
  // an invalid page are left out of the softmax, as in decode, and staged
  // as zeros).
  bool clean;
  const int n_pt = min((n_tiles * KT + P.L.block_tokens - 1) / P.L.block_tokens, k_max_seq_pages);
  {
    int bad = n_pt * P.L.block_tokens < key_end ? 1 : 0;
    for (int i = tid; i < n_pt; i += NT) {
      const uint32_t page = i < P.table_stride ? table[i] : 0xFFFFFFFFu;
      const bool ok = page < static_cast<uint32_t>(P.L.max_blocks);
      s_ptab[i] = ok ? static_cast<uint16_t>(page) : 0xFFFFu;
      bad |= (ok || i * P.L.block_tokens >= key_end) ? 0 : 1;
    }
    clean = __syncthreads_or(bad) == 0;
  }
  // K staging: item -> one 8-half chunk of one key row.  V staging: item ->
  // 4 consecutive keys x 2 dims (dims fastest keeps each key row coalesced),
  // transposed in registers so each dim's 4 keys reach LDS as one 8-byte
  // store in the accumulator's key order.
  using stage_t = prefill_stage<KI, VI, Q8>;
  const uint32_t splane = static_cast<uint32_t>(P.L.block_tokens) * D;  // q8_0 scale plane

  // Page of a key from the LDS copy of this sequence's page list (no
  // dependent global load between a tile's address and its data).
  const int bt = P.L.block_tokens;
  const int bt_shift = P.bt_shift;  // log2(block_tokens), or -1
  // Returns the key's region base (its page, this KV head) and its row.
  auto key_region = [&](int key, uint32_t &ok, uint32_t &row) -> uint64_t {
    const int lb = bt_shift >= 0 ? key >> bt_shift : key / bt;
    row = static_cast<uint32_t>(bt_shift >= 0 ? key & (bt - 1) : key % bt);
    // a sequence holds at most k_max_seq_pages pages (MAX_BLOCKS_PER_SEQUENCE)
    const uint32_t page = (key < total && lb < n_pt) ? s_ptab[lb] : 0xFFFFu;
    ok = page != 0xFFFFu ? 1u : 0u;
    return layer_base + static_cast<uint64_t>(ok ? page : 0u) * P.L.page_bytes;
  };
  // f16: byte offset of the key's row.
  auto key_offset = [&](int key, uint32_t &ok) -> uint64_t {
    uint32_t row;
    return key_region(key, ok, row) + static_cast<uint64_t>(row) * D * 2u;
  };
  // Uniform sub-tiles (block_tokens a multiple of 32): each 32-key sub-tile
  // lies in one page, so its base address is wave-uniform and every thread
  // adds fixed offsets; loads are unconditional.  Keys past the sequence end
  // get zero V (their P is 0, and 0 * garbage could be NaN); a sub-tile on an
  // invalid page is all zeros, as the general path gives.
  const bool uniform_tiles = bt_shift >= 5;
  constexpr bool BUF = !Q8 && NT == 4 * D && KI == NS && VI == NS;
  // Offsets inside a 32-key sub-tile (q8_0: of the values, and of the
  // scale of the item's 32-value block from the scale plane).
  uint32_t kofs[KI], vofs[VI], ksofs[KI], vsofs[VI];
  int ksub[KI], vsub[VI];
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int item = tid + i * NT;
    const int key = item / (D / 8);
    const int chunk = item % (D / 8);
    ksub[i] = key / k_sub;
    kofs[i] = static_cast<uint32_t>(key % k_sub) * ROWB + chunk * (ROWB / (D / 8));
    ksofs[i] = static_cast<uint32_t>(key % k_sub) * SROWB + (chunk / 4) * 2;
  }
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int item = tid + i * NT;
    const int key = 4 * (item / (D / 2));
    const int dp = item % (D / 2);
    vsub[i] = key / k_sub;
    vofs[i] = static_cast<uint32_t>(key % k_sub) * ROWB + dp * (ROWB / (D / 2));
    vsofs[i] = static_cast<uint32_t>(key % k_sub) * SROWB + (dp / 16) * 2;
  }
  // Page of each sub-tile of tile t (0xFFFF: invalid or past the end).
  auto tile_pages = [&](int t, uint32_t (&pg)[NS]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int kj = t * KT + j * k_sub;
      const int lb = kj >> bt_shift;
      pg[j] = (kj < total && lb < n_pt) ? static_cast<uint32_t>(s_ptab[lb]) : 0xFFFFu;
    }
  };
  // The BUF path reads the next tile's page ids one tile ahead, so the
  // LDS round trip of the lookup never sits between a tile's start and its
  // loads.
  uint32_t pg_next[NS];
  auto load_tile_uniform = [&](int t, stage_t &R) __attribute__((always_inline)) {
    const int key0 = t * KT;
    if constexpr (BUF) {
      // f16, one staging item of K and of V per thread and sub-tile (NT =
      // 4 * D): item i of every thread lies in sub-tile i.  One buffer
      // resource per sub-tile and pool, based at the sub-tile's first key
      // row (wave-uniform, built on the scalar unit), so each load is that
      // base + a fixed per-thread offset.  An invalid page gets a resource
      // of 0 bytes: its loads return zeros.
      __amdgpu_buffer_rsrc_t krs[NS], vrs[NS];
      bool all_valid = true;
      uint32_t pg[NS];
      if (t == 0) {
        tile_pages(0, pg);
      } else {
#pragma unroll
        for (int j = 0; j < NS; ++j) pg[j] = pg_next[j];
      }
      tile_pages(t + 1, pg_next);
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int kj = key0 + j * k_sub;
        const uint32_t page = __builtin_amdgcn_readfirstlane(pg[j]);
        const bool valid = page != 0xFFFFu;
        all_valid = all_valid && valid;
        const uint64_t off = layer_base + static_cast<uint64_t>(valid ? page : 0u) * P.L.page_bytes +
                             static_cast<uint64_t>(kj & (bt - 1)) * ROWB;
        const int bytes = valid ? static_cast<int>(k_sub * ROWB) : 0;
        krs[j] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(P.k_pool + off), 0, bytes,
                                                   k_rsrc_word3);
        vrs[j] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(P.v_pool + off), 0, bytes,
                                                   k_rsrc_word3);
      }
#pragma unroll
      for (int i = 0; i < KI; ++i) {
        if (KITEMS % NT == 0 || tid + i * NT < KITEMS) {
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(krs[i], static_cast<int>(kofs[i]), 0, 0);
          R.rk[i] = uint4_t{v[0], v[1], v[2], v[3]};
        }
      }
#pragma unroll
      for (int i = 0; i < VI; ++i) {
        if (VITEMS % NT == 0 || tid + i * NT < VITEMS) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            R.rv[i][e] = __builtin_amdgcn_raw_buffer_load_b32(
                vrs[i], static_cast<int>(vofs[i] + e * ROWB), 0, 0);
          }
        }
      }
      (void)all_valid;
      if (key0 + KT > total) {  // keys past the end: zero V (P is 0 there; 0 * NaN is not)
#pragma unroll
        for (int i = 0; i < VI; ++i) {
          const int k4 = key0 + 4 * ((tid + i * NT) / (D / 2));
#pragma unroll
          for (int e = 0; e < 4; ++e) R.rv[i][e] = k4 + e < total ? R.rv[i][e] : 0u;
        }
      }
      return;
    }
    uint64_t base[NS], sbase[NS];  // values, and (q8_0) scales, of each sub-tile's first key
    bool valid[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int kj = key0 + j * k_sub;
      const int lb = kj >> bt_shift;
      const uint32_t page = __builtin_amdgcn_readfirstlane(
          (kj < total && lb < n_pt) ? static_cast<uint32_t>(s_ptab[lb]) : 0xFFFFu);
      valid[j] = page != 0xFFFFu;
      const uint64_t reg = layer_base + static_cast<uint64_t>(valid[j] ? page : 0u) * P.L.page_bytes;
      base[j] = reg + static_cast<uint64_t>(kj & (bt - 1)) * ROWB;
      if constexpr (Q8) sbase[j] = reg + splane + static_cast<uint64_t>(kj & (bt - 1)) * SROWB;
    }
    // Loads are unconditional; the fix-ups below sit behind one uniform
    // branch, so the common path never waits for the data here (a select
    // on the loaded values would force that wait and expose the latency).
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      if (KITEMS % NT == 0 || tid + i * NT < KITEMS) {
        const int j = NS == 1 ? 0 : ksub[i];
        if constexpr (Q8) {
          R.rk[i] = *reinterpret_cast<const uint2_v *>(P.k_pool + (base[j] + kofs[i]));
          R.ks[i] = *reinterpret_cast<const uint16_t *>(P.k_pool + (sbase[j] + ksofs[i]));
        } else {
          R.rk[i] = load16(P.k_pool + (base[j] + kofs[i]));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      if (VITEMS % NT == 0 || tid + i * NT < VITEMS) {
        const int j = NS == 1 ? 0 : vsub[i];
        const uint64_t vb = base[j] + vofs[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (Q8) {
            const uint64_t sb = sbase[j] + vsofs[i];
            const uint32_t q = *reinterpret_cast<const uint16_t *>(P.v_pool + vb + e * ROWB);
            const uint32_t d = *reinterpret_cast<const uint16_t *>(P.v_pool + sb + e * SROWB);
            R.rv[i][e] = q | (d << 16);
          } else {
            R.rv[i][e] = *reinterpret_cast<const uint32_t *>(P.v_pool + vb + e * ROWB);
          }
        }
      }
    }
    bool all_valid = true;
#pragma unroll
    for (int j = 0; j < NS; ++j) all_valid = all_valid && valid[j];
    if (!all_valid || key0 + KT > total) {
#pragma unroll
      for (int i = 0; i < KI; ++i) {
        if (!valid[NS == 1 ? 0 : ksub[i]]) {
          if constexpr (Q8) {
            R.rk[i] = uint2_v{0u, 0u};
            R.ks[i] = 0u;
          } else {
            R.rk[i] = uint4_t{0u, 0u, 0u, 0u};
          }
        }
      }
#pragma unroll
      for (int i = 0; i < VI; ++i) {
        const int j = NS == 1 ? 0 : vsub[i];
        const int k4 = key0 + 4 * ((tid + i * NT) / (D / 2));
#pragma unroll
        for (int e = 0; e < 4; ++e) R.rv[i][e] = (valid[j] && k4 + e < total) ? R.rv[i][e] : 0u;
      }
    }
  };
  auto load_tile_general = [&](int t, stage_t &R) __attribute__((always_inline)) {
    if constexpr (Q8) {
#pragma unroll
      for (int i = 0; i < KI; ++i) {
        const int item = tid + i * NT;
        if (KITEMS % NT == 0 || item < KITEMS) {
          uint32_t ok, row;
          const uint64_t reg = key_region(t * KT + item / (D / 8), ok, row);
          const uint32_t chunk = item % (D / 8);
          R.rk[i] = ok ? *reinterpret_cast<const uint2_v *>(P.k_pool + reg + row * ROWB + chunk * 8u)
                       : uint2_v{0u, 0u};
          R.ks[i] = ok ? *reinterpret_cast<const uint16_t *>(P.k_pool + reg + splane + row * SROWB +
                                                             (chunk / 4) * 2u)
                       : 0u;
        }
      }
#pragma unroll
      for (int i = 0; i < VI; ++i) {
        const int item = tid + i * NT;
        if (VITEMS % NT == 0 || item < VITEMS) {
          const int dp = item % (D / 2);
          const int key0 = t * KT + 4 * (item / (D / 2));
          // the 4 keys share a page whenever block_tokens is a multiple of 4
          const bool same_page = (bt & 3) == 0;
          uint32_t ok0, row0;
          const uint64_t reg0 = key_region(key0, ok0, row0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            uint32_t ok = ok0, row = row0 + j;
            uint64_t reg = reg0;
            if (!same_page) reg = key_region(key0 + j, ok, row);
            ok = ok && (key0 + j < total);
            const uint32_t q =
                ok ? *reinterpret_cast<const uint16_t *>(P.v_pool + reg + row * ROWB + 2u * dp) : 0u;
            const uint32_t d = ok ? *reinterpret_cast<const uint16_t *>(
                                        P.v_pool + reg + splane + row * SROWB + (dp / 16) * 2u)
                                  : 0u;
            R.rv[i][j] = q | (d << 16);
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < KI; ++i) {
        const int item = tid + i * NT;
        if (KITEMS % NT == 0 || item < KITEMS) {
          uint32_t ok;
          const uint64_t off = key_offset(t * KT + item / (D / 8), ok) + (item % (D / 8)) * 16u;
          R.rk[i] = ok ? load16(P.k_pool + off) : uint4_t{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (int i = 0; i < VI; ++i) {
        const int item = tid + i * NT;
        if (VITEMS % NT == 0 || item < VITEMS) {
          const int dp = item % (D / 2);
          const int key0 = t * KT + 4 * (item / (D / 2));
          // the 4 keys share a page whenever block_tokens is a multiple of 4
          const bool same_page = (bt & 3) == 0;
          uint32_t ok0;
          const uint64_t off0 = key_offset(key0, ok0) + 4u * dp;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            uint32_t ok = ok0;
            uint64_t off = off0 + static_cast<uint64_t>(j) * D * 2u;
            if (!same_page) off = key_offset(key0 + j, ok) + 4u * dp;
            ok = ok && (key0 + j < total);
            R.rv[i][j] = ok ? *reinterpret_cast<const uint32_t *>(P.v_pool + off) : 0u;
          }
        }
      }
    }
  };
  auto load_tile = [&](int t, stage_t &R) __attribute__((always_inline)) {
    if (uniform_tiles) {
      load_tile_uniform(t, R);
    } else {
      load_tile_general(t, R);
    }
  };
  auto store_tile = [&](int kbuf, int vbuf, const stage_t &R) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = tid + i * NT;
      if (KITEMS % NT == 0 || item < KITEMS) {
        const int krow = item / (D / 8);
        const int kcol = (item % (D / 8)) * 8;
        if constexpr (Q8) {
          const half2_t d2 = as_half2(R.ks[i] * 0x10001u);
          const uint2_v a = q8_pair_to_f16x2(R.rk[i].x & 0xFFFFu, d2);
          const uint2_v b = q8_pair_to_f16x2(R.rk[i].x >> 16, d2);
          const uint2_v c = q8_pair_to_f16x2(R.rk[i].y & 0xFFFFu, d2);
          const uint2_v e = q8_pair_to_f16x2(R.rk[i].y >> 16, d2);
          *reinterpret_cast<uint4_t *>(&s_k[kbuf][0][krow][kcol]) = uint4_t{a.x, b.x, c.x, e.x};
          *reinterpret_cast<uint4_t *>(&s_k[kbuf][PL - 1][krow][kcol]) = uint4_t{a.y, b.y, c.y, e.y};
        } else {
          *reinterpret_cast<uint4_t *>(&s_k[kbuf][0][krow][kcol]) = R.rk[i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = tid + i * NT;
      if (VITEMS % NT == 0 || item < VITEMS) {
        const int dp = item % (D / 2);
        const int key4 = 4 * (item / (D / 2));  // 4 consecutive keys -> 4 slots
        const int slot = (key4 / k_sub) * k_sub + (M16 ? key_slot16(key4 % k_sub)
                                                        : key_slot(key4 % k_sub));
        // lanes 8..15 of each 16 write their odd row first: the two rows of
        // a lane are 4 banks apart, so each write instruction spreads over
        // twice as many banks (measured: LDS bank-conflict cycles 13.5M ->
        // 4.5M per launch at the Llama-3-8B chunk shape)
        const bool odd_first = (tid & 8) != 0;
        const int r0 = 2 * dp + (odd_first ? 1 : 0);
        // the row written first takes the high halves when it is the odd
        // row: chosen by the permute selector, not by selecting data
        const uint32_t sel_first = odd_first ? 0x07060302u : 0x05040100u;
        const uint32_t sel_second = odd_first ? 0x05040100u : 0x07060302u;
        auto put = [&](int pl, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
          const uint2 first{__builtin_amdgcn_perm(w1, w0, sel_first),
                            __builtin_amdgcn_perm(w3, w2, sel_first)};
          const uint2 second{__builtin_amdgcn_perm(w1, w0, sel_second),
                             __builtin_amdgcn_perm(w3, w2, sel_second)};
          *reinterpret_cast<uint2 *>(&s_vt[vbuf][pl][r0][slot]) = first;
          *reinterpret_cast<uint2 *>(&s_vt[vbuf][pl][r0 ^ 1][slot]) = second;
        };
        if constexpr (Q8) {
          uint2_v w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            w[e] = q8_pair_to_f16x2(R.rv[i][e] & 0xFFFFu, as_half2((R.rv[i][e] >> 16) * 0x10001u));
          }
          put(0, w[0].x, w[1].x, w[2].x, w[3].x);  // hi: fp16(q * d)
          put(PL - 1, w[0].y, w[1].y, w[2].y, w[3].y);  // lo: q * d - hi, exact
        } else {
          put(0, R.rv[i][0], R.rv[i][1], R.rv[i][2], R.rv[i][3]);
        }
      }
    }
  };

  // One tile in three steps: scores (K ring of 2), online softmax, O update
  // (V ring of 3).
  auto qk = [&](int t, float16_v (&s)[NS]) {
    const int buf = t & 1;
    // S^T = K . Q^T, one accumulator per 32-key sub-tile (independent chains)
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[j][r] = 0.0f;
    }
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
      for (int pl = 0; pl < PL; ++pl) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          const half8_v a = *reinterpret_cast<const half8_v *>(
              &s_k[buf][pl][j * k_sub + l32][16 * kk + 8 * h]);
          s[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qop[kk], s[j], 0, 0, 0);
        }
      }
    }
    if constexpr (NS > 1 && Q8) {
      // operand reads just ahead of their MFMAs rather than all hoisted,
      // which would need 4 * NS * KSTEPS * PL registers at once
#pragma unroll
      for (int kk = 0; kk < KSTEPS * PL; ++kk) {
        __builtin_amdgcn_sched_group_barrier(0x100, NS, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, NS, 0);
      }
    } else if constexpr (NS > 1) {
      // f16: the operand reads run two k-steps ahead of their MFMAs (one
      // step ahead left the LDS latency exposed: 3% slower at the
      // Llama-3-8B chunk shape)
      constexpr int LA = 2;
      __builtin_amdgcn_sched_group_barrier(0x100, LA * NS, 0);
#pragma unroll
      for (int kk = 0; kk < KSTEPS - LA; ++kk) {
        __builtin_amdgcn_sched_group_barrier(0x008, NS, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, NS, 0);
      }
#pragma unroll
      for (int kk = 0; kk < LA; ++kk) __builtin_amdgcn_sched_group_barrier(0x008, NS, 0);
    }
  };
  // Max / sum of v and the value 32 lanes apart, by v_permlane32_swap: with
  // both operands v the two results are v's low and high halves, so every
  // lane gets the same (commutative) combination.
  auto halves = [](float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                    __builtin_bit_cast(uint32_t, v), false, false);
    return float2{__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
                  __builtin_bit_cast(float, static_cast<uint32_t>(r[1]))};
  };
  // Online softmax for query my_row (16 keys in-lane + the other half).
  // INTERIOR tiles lie wholly before the workgroup's first query position
  // and inside the sequence, on valid pages: no mask.
  auto softmax = [&]<bool INTERIOR>(int t, float16_v (&s)[NS]) {
    float tmax = -INFINITY;
    if constexpr (INTERIOR) {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[j][r]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = t * KT + j * k_sub + 8 * (r / 4) + 4 * h + (r % 4);
          s[j][r] = (key <= my_pos && key < total) ? s[j][r] : -INFINITY;
        }
      }
      if (!clean) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = t * KT + j * k_sub + 8 * (r / 4) + 4 * h + (r % 4);
            const int lb = bt_shift >= 0 ? key >> bt_shift : key / bt;
            const bool ok = lb < n_pt && s_ptab[lb] != 0xFFFFu;
            s[j][r] = ok ? s[j][r] : -INFINITY;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < NS; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[j][r]);
      }
    }
    {
      const float2 hv = halves(tmax);
      tmax = fmaxf(hv.x, hv.y);
    }
    const bool need = tmax > m + rescale_raw;
    float alpha = 1.0f;
    if (need) {
      alpha = fast_exp2((m - tmax) * P.c);  // 0 while the row had no valid key yet
      l *= alpha;
      m = tmax;
    }
    const float mc = m * P.c;
    float ps8[8];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(fmaf(s[j][r], P.c, -mc));
        if constexpr (INTERIOR) {  // every score finite, m finite
          s[j][r] = pr;
        } else {
          s[j][r] = s[j][r] == -INFINITY ? 0.0f : pr;  // also covers m == -inf
        }
      }
      // pairwise partial sums: short dependency chains
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float pair = s[j][2 * r] + s[j][2 * r + 1];
        ps8[r] = j == 0 ? pair : ps8[r] + pair;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) ps8[r] += ps8[r + 4];
    float psum = (ps8[0] + ps8[2]) + (ps8[1] + ps8[3]);
    {
      const float2 hv = halves(psum);
      psum = hv.x + hv.y;
    }
    l += psum;

    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      // alpha of each O row: rows 8a + 4h + b live in lane (row), so pass
      // them through LDS (wave-private slice)
      if (h == 0) s_row[wave][l32] = alpha;
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the write lands before the reads
      __builtin_amdgcn_wave_barrier();
      float arow[16];
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const float4_t v = *reinterpret_cast<const float4_t *>(&s_row[wave][8 * a4 + 4 * h]);
        arow[4 * a4 + 0] = v.x;
        arow[4 * a4 + 1] = v.y;
        arow[4 * a4 + 2] = v.z;
        arow[4 * a4 + 3] = v.w;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int c = 0; c < DCH; ++c) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[c][r] *= arow[r];
      }
    }

  };
  auto pv = [&](int t, const float16_v (&s)[NS]) {
    const int buf = t % VR;
    // O += P . V; each fp16 P operand is built right before its four
    // MFMAs (one per 32-dim chunk of O, independent accumulators)
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        half8_v pa;
        [[maybe_unused]] half8_v pl;  // q8_0: P - fp16(P), so hi + lo carries P to about 2^-22
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pa[i] = static_cast<half_t>(s[j][8 * st + i]);
          if constexpr (Q8) pl[i] = static_cast<half_t>(s[j][8 * st + i] - static_cast<float>(pa[i]));
        }
#pragma unroll
        for (int c = 0; c < DCH; ++c) {
          const half8_v b = *reinterpret_cast<const half8_v *>(
              &s_vt[buf][0][32 * c + l32][j * k_sub + 16 * st + 8 * h]);
          o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, b, o[c], 0, 0, 0);
          if constexpr (Q8) {
            // P_hi V_lo + P_lo V_hi; P_lo V_lo (about 2^-22 of P V) is left out
            const half8_v bl = *reinterpret_cast<const half8_v *>(
                &s_vt[buf][PL - 1][32 * c + l32][j * k_sub + 16 * st + 8 * h]);
            o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, bl, o[c], 0, 0, 0);
            o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl, b, o[c], 0, 0, 0);
          }
        }
      }
    }
    {
      // the V operand reads run four MFMAs ahead (measured 2% faster than
      // the compiler's own order at the Llama-3-8B chunk shape)
      // (q8_0: per operand pair, 2 reads and 3 MFMAs)
      constexpr int NPV = NS * 2 * DCH;
      constexpr int LAP = 4;
      constexpr int RD = Q8 ? 2 : 1, MF = Q8 ? 3 : 1;
      __builtin_amdgcn_sched_group_barrier(0x100, LAP * RD, 1);
#pragma unroll
      for (int k = 0; k < NPV - LAP; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, MF, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, RD, 1);
      }
#pragma unroll
      for (int k = 0; k < LAP; ++k) __builtin_amdgcn_sched_group_barrier(0x008, MF, 1);
    }
  };

  // Single register stage: tile t + 1 is loaded at the start of tile t and
  // written to the free LDS buffers after tile t's work.  Deeper register
  // rings, and a software pipeline issuing tile t+1's QK MFMAs before tile
  // t's softmax within one wave, were both measured slower: their unrolled
  // copies push the kernel past 256 registers per lane, the budget at 8
  // waves per CU (the pipeline, with K staged two tiles ahead, a ring of 3
  // V buffers and sched_group_barrier interleaving, still spilled 18
  // registers and ran at 512 vs 809 TFLOP/s).  Staging K by direct
  // global->LDS loads (XOR-swizzled rows, issued after the tile's QK reads
  // so no LDS read waits on them) was correct but slower: 744 TFLOP/s at
  // 32-key tiles; at 64-key tiles it spills, and every scratch reload then
  // waits on the in-flight loads.
  //
  // Tried and measured slower on MI355X: running the two waves that share a
  // SIMD half a tile apart (one in softmax while the other issues MFMAs,
  // with a ring of 3 V buffers), 700 vs 758 TFLOP/s; and two 4-wave
  // workgroups per CU instead of one 8-wave workgroup, 2.6x slower.
  // Four waves of 64 query rows each (one wave per SIMD, so each K or V
  // operand read from LDS feeds two MFMAs and 512 registers are available)
  // was correct but ran at 141 TFLOP/s: the compiler keeps the score
  // accumulators in AGPRs, copies them through VGPRs for the softmax and
  // spills the staging state to scratch.  With 32-key tiles it compiles
  // without spills but runs at 529 vs 823 TFLOP/s: one wave per SIMD leaves
  // nothing to issue MFMAs while a wave is in its softmax, and the
  // accumulators still move between AGPRs and VGPRs on every tile.
  // Staging V key-major (16-byte stores, no register transpose) and reading
  // the P.V operand with LDS transpose loads (ds_read_b64_tr_b16, two per
  // operand) was correct but slower: 779 vs 824 TFLOP/s with rows padded to
  // D + 32 halves, 736 with D + 8.
  // A software pipeline with 32-key tiles (tile t+1's scores computed in the
  // same stretch as tile t's softmax, K staged two tiles ahead, a ring of 3
  // V buffers, 228 VGPRs): 812 vs 826 TFLOP/s, and 790 with the K reads and
  // MFMAs explicitly interleaved into the softmax (sched_group_barrier).
  // The online softmax per 32-key sub-tile, so that sub-tile 1's score
  // MFMAs and sub-tile 0's P.V MFMAs could issue beside the other
  // sub-tile's softmax (240 VGPRs, no spills): 374 vs 357 us per launch
  // at the Llama-3-8B chunk shape with the compiler's own order, and 391
  // with sched_group_barrier interleaving (q8_0: 627 and 644 vs 621).
  // Q^T kept in LDS instead of registers (225 instead of 256 VGPRs, one
  // more LDS operand read per k-step): 801 vs 834 TFLOP/s.  Four waves of
  // 32 rows (the head_dim 256 layout) at head_dim 128: 490 vs 810.  At
  // head_dim 256 (one wave per SIMD), the next tile's scores computed in
  // the same stretch as this tile's softmax, K and V staged two tiles ahead
  // in rings of 3: 458-463 vs 488 TFLOP/s.
  // ---- M16 (16 rows per wave, v_mfma_f32_16x16x32_f16) ----
  // S^T tile j (16 keys) = K (16 x D) . Q^T (D x 16): lane l holds keys
  // 16j + 4*g16 + r (r < 4) of query row c16; the row's other 24 scores
  // sit in the lanes 16, 32 and 48 apart.
  auto qk16 = [&](int t, float4_v (&s)[2]) {
    const int buf = t & 1;
    s[0] = float4_v{0.0f, 0.0f, 0.0f, 0.0f};
    s[1] = s[0];
#pragma unroll
    for (int kk = 0; kk < KS16; ++kk) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const half8_v a =
            *reinterpret_cast<const half8_v *>(&s_k[buf][0][16 * j + c16][32 * kk + 8 * g16]);
        s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qop16[kk], s[j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int kk = 0; kk < KS16; ++kk) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
  };
  // Max / sum over the four lanes of a query row (lanes 16 apart).
  auto row4_max = [](float v) {
    v = fmaxf(v, __shfl_xor(v, 16, k_wave));
    return fmaxf(v, __shfl_xor(v, 32, k_wave));
  };
  auto row4_sum = [](float v) {
    v += __shfl_xor(v, 16, k_wave);
    return v + __shfl_xor(v, 32, k_wave);
  };
  auto softmax16 = [&]<bool INTERIOR>(int t, float4_v (&s)[2]) {
    if constexpr (!INTERIOR) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = t * KT + 16 * j + 4 * g16 + r;
          bool ok = key <= my_pos && key < total;
          if (!clean) {
            const int lb = bt_shift >= 0 ? key >> bt_shift : key / bt;
            ok = ok && lb < n_pt && s_ptab[lb] != 0xFFFFu;
          }
          s[j][r] = ok ? s[j][r] : -INFINITY;
        }
      }
    }
    float tmax = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                       fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    tmax = row4_max(tmax);
    const bool need = tmax > m + rescale_raw;
    float alpha = 1.0f;
    if (need) {
      alpha = fast_exp2((m - tmax) * P.c);  // 0 while the row had no valid key yet
      l *= alpha;
      m = tmax;
    }
    const float mc = m * P.c;
    float psum = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = fast_exp2(fmaf(s[j][r], P.c, -mc));
        s[j][r] = (INTERIOR || s[j][r] != -INFINITY) ? pr : 0.0f;
      }
      psum += (s[j][0] + s[j][1]) + (s[j][2] + s[j][3]);
    }
    l += row4_sum(psum);
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      // alpha of the O rows 4*g16 + r of this lane: from the lanes that own
      // those query rows, through LDS (wave-private slice)
      if (g16 == 0) s_row[wave][c16] = alpha;
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      const float4_t ar = *reinterpret_cast<const float4_t *>(&s_row[wave][4 * g16]);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int c = 0; c < OT16; ++c) {
        o16[c][0] *= ar.x;
        o16[c][1] *= ar.y;
        o16[c][2] *= ar.z;
        o16[c][3] *= ar.w;
      }
    }
  };
  // O (16 rows x D) += P (16 x 32 keys) . V (32 x D); the P operand of lane l
  // is its own 8 probabilities, in the slot order the V^T staging used.
  auto pv16 = [&](int t, const float4_v (&s)[2]) {
    const int buf = t % VR;
    half8_v pa;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pa[r] = static_cast<half_t>(s[0][r]);
      pa[4 + r] = static_cast<half_t>(s[1][r]);
    }
#pragma unroll
    for (int c = 0; c < OT16; ++c) {
      const half8_v b =
          *reinterpret_cast<const half8_v *>(&s_vt[buf][0][16 * c + c16][8 * g16]);
      o16[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, b, o16[c], 0, 0, 0);
    }
  };

  stage_t R;
  load_tile(0, R);
  store_tile(0, 0, R);
  __syncthreads();
  float16_v s[NS];
  // tiles [0, n_int) need no mask
  const int n_int = clean ? min(n_tiles, min((wg_first_pos + 1) / KT, total / KT)) : 0;
  float4_v s16[2];
  auto step = [&]<bool INTERIOR>(int t) {
    const bool more = t + 1 < n_tiles;
    if (more) load_tile(t + 1, R);
    if constexpr (M16) {
      qk16(t, s16);
      softmax16.template operator()<INTERIOR>(t, s16);
      pv16(t, s16);
    } else {
      qk(t, s);
      softmax.template operator()<INTERIOR>(t, s);
      pv(t, s);
    }
    if (more) store_tile((t + 1) & 1, (t + 1) % VR, R);
    __syncthreads();
  };
  for (int t = 0; t < n_int; ++t) step.template operator()<true>(t);
  for (int t = n_int; t < n_tiles; ++t) step.template operator()<false>(t);

  // normalise by l of each row and write rows < n_q
  if constexpr (M16) {
    __builtin_amdgcn_wave_barrier();
    if (g16 == 0) s_row[wave][c16] = l > 0.0f ? 1.0f / l : 0.0f;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    const float4_t inv = *reinterpret_cast<const float4_t *>(&s_row[wave][4 * g16]);
    const float invs[4] = {inv.x, inv.y, inv.z, inv.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 4 * g16 + r;
      if (row >= n_q) continue;
      float *op = P.out + ((static_cast<uint64_t>(seq) * n_q + row) * P.L.n_head + head) * D;
#pragma unroll
      for (int c = 0; c < OT16; ++c) op[16 * c + c16] = o16[c][r] * invs[r];
    }
    return;
  }
  __builtin_amdgcn_wave_barrier();
  if (h == 0) s_row[wave][l32] = l > 0.0f ? 1.0f / l : 0.0f;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = row0 + 8 * (r / 4) + 4 * h + (r % 4);
    if (row >= n_q) continue;
    const float inv = s_row[wave][8 * (r / 4) + 4 * h + (r % 4)];
    float *op = P.out + ((static_cast<uint64_t>(seq) * n_q + row) * P.L.n_head + head) * D;
#pragma unroll
    for (int c = 0; c < DCH; ++c) op[32 * c + l32] = o[c][r] * inv;
  }
}

template <int D, int KT, bool Q8, bool M16 = false>
bool launch_prefill_kt(const prefill_params &P, int32_t n_seq, hipStream_t st) {
  // W waves per workgroup: G_WG query heads of one KV group x RB blocks of
  // 32 query rows, all sharing each staged K/V tile.  head_dim 256 runs 4
  // waves, one per SIMD, so each has the full register file for its 32 x
  // 256 O tile and Q^T operand (8 waves at head_dim <= 128).
  constexpr int W = D > 128 ? 4 : 8;
  static_assert(!M16 || W == 4, "M16 runs 4 waves per workgroup");
  const int group = P.L.n_head / P.L.n_head_kv;
  const int g_wg = group < W ? group : W;
  const int rb = W / g_wg;
  constexpr int ROWS = M16 ? 16 : 32;
  const int n_qt = (P.n_q + ROWS * rb - 1) / (ROWS * rb);
  const dim3 grid(n_qt * (P.L.n_head / g_wg) * n_seq);
  const dim3 block(W * k_wave);
  switch (g_wg) {
    case 1: hipLaunchKernelGGL((prefill_kernel<D, 1, W, KT, Q8, M16>), grid, block, 0, st, P); return true;
    case 2: hipLaunchKernelGGL((prefill_kernel<D, 2, W / 2, KT, Q8, M16>), grid, block, 0, st, P); return true;
    case 4: hipLaunchKernelGGL((prefill_kernel<D, 4, W / 4, KT, Q8, M16>), grid, block, 0, st, P); return true;
    case 8:
      if constexpr (W == 8) {
        hipLaunchKernelGGL((prefill_kernel<D, 8, 1, KT, Q8, M16>), grid, block, 0, st, P);
        return true;
      }
      return false;
    default: return false;
  }
}

// 64-key tiles: two independent score chains per wave and half the
// barriers of 32-key tiles (measured 834 vs 802 TFLOP/s at the Llama-3-8B
// chunk shape).
constexpr int k_key_tile = 64;

template <int D>
bool launch_prefill(const prefill_params &P, int32_t n_seq, hipStream_t st) {
  if (P.L.kv_type == EMELK_KV_Q8_0) return launch_prefill_kt<D, k_key_tile, true>(P, n_seq, st);
  return launch_prefill_kt<D, k_key_tile, false>(P, n_seq, st);
}

}  // namespace
}  // namespace emelk

extern "C" emel_error_type emelk_attn_prefill_chunk(const emelk_kv_geometry *g, const void *k_pool,
                                                    const void *v_pool, int32_t layer,
                                                    const float *q, float *out, int32_t n_seq,
                                                    int32_t n_q, const int32_t *q_start,
                                                    const uint16_t *block_tables,
                                                    int32_t table_stride, float scale,
                                                    void *stream) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE ||
      k_pool == nullptr || v_pool == nullptr || q == nullptr || out == nullptr ||
      q_start == nullptr || block_tables == nullptr || layer < 0 || layer >= L.n_layer ||
      n_seq <= 0 || n_seq > 65535 || n_q <= 0 || table_stride <= 0 || !(scale > 0.0f) ||
      !std::isfinite(scale)) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  if (L.head_dim == 512 && L.kv_type == EMELK_KV_Q8_0) {
    // q8_0 at head_dim 512: row by row through the decode kernel, as the
    // reference's per-row loop does (K's hi/lo planes do not fit the LDS).
    // f16 pools at 512 run 16 query rows per wave (M16): a wave's 32 x 512
    // O tile and Q^T operand take 384 of its 512 registers, and built that
    // way the kernel spills about 1500 registers per lane (about 350 with
    // wave pairs that split O's columns).
    return emelk::decode_rows(L, k_pool, v_pool, layer, q, out, n_seq, n_q, q_start,
                              block_tables, table_stride, scale, static_cast<hipStream_t>(stream));
  }
  emelk::prefill_params P;
  P.L = L;
  P.k_pool = static_cast<const uint8_t *>(k_pool);
  P.v_pool = static_cast<const uint8_t *>(v_pool);
  P.layer = layer;
  P.q = q;
  P.out = out;
  P.n_q = n_q;
  P.q_start = q_start;
  P.tables = block_tables;
  P.table_stride = table_stride;
  P.c = scale * 1.4426950408889634f;
  P.bt_shift = -1;
  for (int b = 0; b < 16; ++b) {
    if ((1 << b) == L.block_tokens) P.bt_shift = b;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool q8 = L.kv_type == EMELK_KV_Q8_0;
  // head_dim 256: 32-key tiles (64 spill, and q8_0's hi/lo K planes of
  // 64-key tiles would not fit the LDS)
  const bool ok = L.head_dim == 512 ? emelk::launch_prefill_kt<512, 32, false, true>(P, n_seq, st)
                  : L.head_dim == 256
                      ? (q8 ? emelk::launch_prefill_kt<256, 32, true>(P, n_seq, st)
                            : emelk::launch_prefill_kt<256, 32, false>(P, n_seq, st))
                  : L.head_dim == 128 ? emelk::launch_prefill<128>(P, n_seq, st)
                                      : emelk::launch_prefill<64>(P, n_seq, st);
  if (!ok) return EMELK_ERR_INVALID_REQUEST;
  return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
}
