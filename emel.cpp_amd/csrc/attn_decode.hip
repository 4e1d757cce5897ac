// Split-K flash-decode GQA attention over the paged pool (gfx950, wave64).
//
// Replaces the reference's paged decode route compute_attention
// (text/generator/detail.hpp:3153-3230) and its contiguous flash route
// (kernel/detail.hpp:5238-5291) with one kernel family:
//
//   grid  = (split, kv_head, sequence); 256 threads = 4 waves.
//   Each workgroup streams the K and V rows of its context slice once from
//   HBM and serves all G = n_head/n_head_kv query heads of its KV head with
//   them (GQA sharing).  A row of D halves is split over L = D/16 lanes
//   (32 bytes = two 16-byte loads per lane); the 256/L lane groups each own
//   two tokens of every 2*256/L-token tile and keep an fp32 online-softmax
//   state (m, l, acc) per head.  Scores: v_dot2_f32_f16 on fp16 q (q is
//   rounded to fp16 as round_q_for_nonflash does, detail.hpp:2898-2903) and
//   a DPP sum over the L lanes.  P.V: v_dot2_f32_f16 of the fp16 pair
//   (p_t0, p_t1) against the paired V values of the two tokens (the
//   reference also rounds probabilities to fp16, detail.hpp:3146-3149).
//   The next tile's rows are loaded before the current tile is used.
//   At the end the groups are merged by wave shuffles and an LDS pass, and
//   one partial (m, l, acc[D]) per (sequence, head, split) is written.
//   A second kernel merges the splits.
//
// q8_0 pools: identical structure; for scores the 16 int8 values of a lane
// are turned into exact fp16 with a byte-permute + packed subtract and the
// lane's block scale multiplies its partial score; for P.V the int8 values
// go to fp32 and the token scale folds into an fp32 weight p * d_v.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>

#include "device_common.hpp"
#include "emelk.h"
#include "pool_layout.hpp"

namespace emelk {
namespace {

using namespace emelk::dev;

constexpr int k_threads = 256;
constexpr int k_waves = k_threads / k_wave;
constexpr int k_max_split_pages = 1024;

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
};

// 16 int8 -> 8 exact half2: byte b becomes the fp16 bit pattern 0x64XX with
// XX = b + 128 (value 1024 + b + 128), then 1152 is subtracted.
__device__ __forceinline__ void i8x16_to_half(const uint4_t w, half2_t out[8]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  const half2_t bias = {static_cast<half_t>(1152.0f), static_cast<half_t>(1152.0f)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = ws[i] ^ 0x80808080u;
    out[2 * i] = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
    out[2 * i + 1] = as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
  }
}

// 16 int8 -> 16 fp32 (exact).
__device__ __forceinline__ void i8x16_to_float(const uint4_t w, float out[16]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      out[4 * i + b] = static_cast<float>(static_cast<int8_t>((ws[i] >> (8 * b)) & 0xFFu));
    }
  }
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

template <int D, bool Q8>
__device__ __forceinline__ void load_row(const uint8_t *__restrict__ region_base, int32_t off,
                                         int32_t dim0, int32_t bt, row_regs<D, Q8> &r) {
  if constexpr (!Q8) {
    const uint8_t *p = region_base + (static_cast<uint64_t>(off) * D + dim0) * 2u;
    r.a = load16(p);
    r.b = load16(p + 16);
  } else {
    r.a = load16(region_base + static_cast<uint64_t>(off) * D + dim0);
    const uint16_t *sc = reinterpret_cast<const uint16_t *>(region_base + static_cast<uint64_t>(bt) * D);
    r.d = sc[off * (D / 32) + dim0 / 32];
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
    i8x16_to_half(r.a, h);
    scale = f16_bits_to_f32(static_cast<uint16_t>(r.d));
  }
}

template <int D, int G, bool Q8>
__global__ __launch_bounds__(k_threads, 2) void decode_kernel(decode_params P) {
  constexpr int LPT = D / 16;           // lanes per token row
  constexpr int NG = k_threads / LPT;   // token groups per workgroup
  constexpr int TT = 2 * NG;            // tokens per tile

  __shared__ uint32_t s_pages[k_max_split_pages];
  __shared__ float s_acc[k_waves][G][D];
  __shared__ float s_ml[k_waves][G][2];

  const int32_t split = blockIdx.x;
  const int32_t kvh = blockIdx.y;
  const int32_t seq = blockIdx.z;
  const int32_t tid = threadIdx.x;
  const int32_t len = P.kv_lens[seq];
  const int32_t start = split * P.tokens_per_split;
  if (start >= len) return;  // the combine kernel never reads this split
  const int32_t end = min(len, start + P.tokens_per_split);
  const int32_t bt = P.L.block_tokens;
  const int32_t first_page = start / bt;
  const int32_t n_pages = (end - 1) / bt - first_page + 1;

  const uint16_t *table = P.tables + static_cast<uint64_t>(seq) * P.table_stride;
  for (int32_t i = tid; i < n_pages; i += k_threads) {
    const int32_t lb = first_page + i;
    const uint32_t page = lb < P.table_stride ? table[lb] : 0xFFFFFFFFu;
    s_pages[i] = page < static_cast<uint32_t>(P.L.max_blocks) ? page : 0xFFFFFFFFu;
  }

  const int32_t lane_in_row = tid % LPT;
  const int32_t grp = tid / LPT;
  const int32_t dim0 = lane_in_row * 16;
  const uint64_t layer_base = static_cast<uint64_t>(P.layer) * P.L.layer_bytes +
                              static_cast<uint64_t>(kvh) * P.L.region_bytes;

  // q for the G heads of this KV head, rounded to fp16.
  half2_t qh[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float *qp = P.q + (static_cast<uint64_t>(seq) * P.L.n_head + kvh * G + h) * D + dim0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4_t f = reinterpret_cast<const float4_t *>(qp)[j];
      qh[h][2 * j] = pack_half2(f.x, f.y);
      qh[h][2 * j + 1] = pack_half2(f.z, f.w);
    }
  }

  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[h][i] = 0.0f;
  }
  __syncthreads();

  // Byte offset of the page holding token `tok` (tok already clamped into
  // the split by the caller).  Invalid pages read page 0 and are masked.
  auto page_off = [&](int32_t tok, bool &ok) -> uint64_t {
    const uint32_t page = s_pages[tok / bt - first_page];
    const bool valid = page != 0xFFFFFFFFu;
    ok = ok && valid;
    return layer_base + static_cast<uint64_t>(valid ? page : 0u) * P.L.page_bytes;
  };
  auto load_pair = [&](int32_t tbase, bool &okA, bool &okB, row_regs<D, Q8> &ka,
                       row_regs<D, Q8> &kb, row_regs<D, Q8> &va, row_regs<D, Q8> &vb) {
    okA = tbase + grp < end;
    okB = tbase + grp + NG < end;
    const int32_t t0 = okA ? tbase + grp : start;
    const int32_t t1 = okB ? tbase + grp + NG : start;
    const uint64_t r0 = page_off(t0, okA);
    const uint64_t r1 = page_off(t1, okB);
    load_row<D, Q8>(P.k_pool + r0, t0 % bt, dim0, bt, ka);
    load_row<D, Q8>(P.k_pool + r1, t1 % bt, dim0, bt, kb);
    load_row<D, Q8>(P.v_pool + r0, t0 % bt, dim0, bt, va);
    load_row<D, Q8>(P.v_pool + r1, t1 % bt, dim0, bt, vb);
  };

  row_regs<D, Q8> k0, k1, v0, v1;
  bool ok0, ok1;
  load_pair(start, ok0, ok1, k0, k1, v0, v1);

  for (int32_t base = start; base < end; base += TT) {
    // prefetch the next tile
    const int32_t nbase = base + TT;
    row_regs<D, Q8> nk0, nk1, nv0, nv1;
    bool nok0 = false, nok1 = false;
    if (nbase < end) load_pair(nbase, nok0, nok1, nk0, nk1, nv0, nv1);

    // scores
    half2_t kh0[8], kh1[8];
    float ks0, ks1;
    to_half<D, Q8>(k0, kh0, ks0);
    to_half<D, Q8>(k1, kh1, ks1);
    float s0[G], s1[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float a = 0.0f, b = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a = dot2(qh[h][j], kh0[j], a);
        b = dot2(qh[h][j], kh1[j], b);
      }
      if constexpr (Q8) {
        a *= ks0;
        b *= ks1;
      }
      s0[h] = group_sum<LPT>(a);
      s1[h] = group_sum<LPT>(b);
    }

    // P.V.  f16 pools: V values of the two tokens paired per dimension and
    // contracted with the fp16 pair (p0, p1) by v_dot2_f32_f16.  q8_0 pools:
    // the int8 values are exact in fp32 and the per-token scale folds into
    // an fp32 weight p*d_v, so nothing is rounded to fp16 (an fp16 p*d_v
    // would cost up to ~2^-11 * 127 * d_v per dominant token).
    [[maybe_unused]] half2_t vlo[8], vhi[8];
    [[maybe_unused]] float vf0[16], vf1[16];
    [[maybe_unused]] float vs0 = 1.0f, vs1 = 1.0f;
    if constexpr (!Q8) {
      half2_t vh0[8], vh1[8];
      to_half<D, Q8>(v0, vh0, vs0);
      to_half<D, Q8>(v1, vh1, vs1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        vlo[j] = as_half2(__builtin_amdgcn_perm(as_u32(vh1[j]), as_u32(vh0[j]), 0x05040100u));
        vhi[j] = as_half2(__builtin_amdgcn_perm(as_u32(vh1[j]), as_u32(vh0[j]), 0x07060302u));
      }
    } else {
      i8x16_to_float(v0.a, vf0);
      i8x16_to_float(v1.a, vf1);
      vs0 = f16_bits_to_f32(static_cast<uint16_t>(v0.d));
      vs1 = f16_bits_to_f32(static_cast<uint16_t>(v1.d));
    }

#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float x0 = ok0 ? s0[h] : -INFINITY;
      const float x1 = ok1 ? s1[h] : -INFINITY;
      const float mn = fmaxf(m[h], fmaxf(x0, x1));
      const float ms = mn == -INFINITY ? 0.0f : mn;
      const float alpha = fast_exp2((m[h] - ms) * P.c);
      const float p0 = fast_exp2((x0 - ms) * P.c);
      const float p1 = fast_exp2((x1 - ms) * P.c);
      l[h] = l[h] * alpha + (p0 + p1);
      m[h] = mn;
      if (alpha != 1.0f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[h][i] *= alpha;
      }
      if constexpr (Q8) {
        const float w0 = p0 * vs0;
        const float w1 = p1 * vs1;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[h][i] = fmaf(w1, vf1[i], fmaf(w0, vf0[i], acc[h][i]));
      } else {
        const half2_t pp = pack_half2(p0, p1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          acc[h][2 * j] = dot2(pp, vlo[j], acc[h][2 * j]);
          acc[h][2 * j + 1] = dot2(pp, vhi[j], acc[h][2 * j + 1]);
        }
      }
    }

    k0 = nk0;
    k1 = nk1;
    v0 = nv0;
    v1 = nv1;
    ok0 = nok0;
    ok1 = nok1;
  }

  // merge the token groups of each wave (lane bits >= log2(LPT))
#pragma unroll
  for (int mask = LPT; mask < k_wave; mask <<= 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mo = wave_shfl_xor(m[h], mask);
      const float lo = wave_shfl_xor(l[h], mask);
      const float mn = fmaxf(m[h], mo);
      const float ms = mn == -INFINITY ? 0.0f : mn;
      const float a = fast_exp2((m[h] - ms) * P.c);
      const float b = fast_exp2((mo - ms) * P.c);
      l[h] = l[h] * a + lo * b;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[h][i] = acc[h][i] * a + wave_shfl_xor(acc[h][i], mask) * b;
      m[h] = mn;
    }
  }
  const int32_t wave = tid / k_wave;
  if ((tid % k_wave) < LPT) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s_acc[wave][h][dim0 + i] = acc[h][i];
      if (lane_in_row == 0) {
        s_ml[wave][h][0] = m[h];
        s_ml[wave][h][1] = l[h];
      }
    }
  }
  __syncthreads();
  for (int32_t idx = tid; idx < G * D; idx += k_threads) {
    const int32_t h = idx / D;
    const int32_t d = idx % D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < k_waves; ++w) mx = fmaxf(mx, s_ml[w][h][0]);
    const float ms = mx == -INFINITY ? 0.0f : mx;
    float lsum = 0.0f, asum = 0.0f;
#pragma unroll
    for (int w = 0; w < k_waves; ++w) {
      const float f = fast_exp2((s_ml[w][h][0] - ms) * P.c);
      lsum += s_ml[w][h][1] * f;
      asum += s_acc[w][h][d] * f;
    }
    const uint64_t slot =
        (static_cast<uint64_t>(seq) * P.L.n_head + kvh * G + h) * P.max_splits + split;
    P.part_acc[slot * D + d] = asum;
    if (d == 0) {
      P.part_ml[slot * 2] = mx;
      P.part_ml[slot * 2 + 1] = lsum;
    }
  }
}

// Merges the split partials of one (sequence, head): o = sum_s e^{m_s-M} acc_s
// / sum_s e^{m_s-M} l_s.
template <int D>
__global__ __launch_bounds__(D) void combine_kernel(const float *__restrict__ part_acc,
                                                     const float *__restrict__ part_ml,
                                                     const int32_t *__restrict__ kv_lens,
                                                     int32_t n_head, int32_t max_splits,
                                                     int32_t tokens_per_split, float c,
                                                     float *__restrict__ out) {
  const int32_t row = blockIdx.x;  // seq * n_head + head
  const int32_t seq = row / n_head;
  const int32_t d = threadIdx.x;
  const int32_t len = kv_lens[seq];
  const int32_t n = len > 0 ? min(max_splits, (len + tokens_per_split - 1) / tokens_per_split) : 0;
  const float *ml = part_ml + static_cast<uint64_t>(row) * max_splits * 2;
  const float *pa = part_acc + static_cast<uint64_t>(row) * max_splits * D;
  float mx = -INFINITY;
  for (int32_t s = 0; s < n; ++s) mx = fmaxf(mx, ml[2 * s]);
  const float ms = mx == -INFINITY ? 0.0f : mx;
  float lsum = 0.0f, asum = 0.0f;
  for (int32_t s = 0; s < n; ++s) {
    const float f = fast_exp2((ml[2 * s] - ms) * c);
    lsum += ml[2 * s + 1] * f;
    asum += pa[static_cast<uint64_t>(s) * D + d] * f;
  }
  out[static_cast<uint64_t>(row) * D + d] = lsum > 0.0f ? asum / lsum : 0.0f;
}

struct decode_plan {
  int32_t tokens_per_split = 0;
  int32_t max_splits = 0;
  uint64_t workspace_bytes = 0;
};

int32_t env_int(const char *name, int32_t fallback) {
  const char *v = std::getenv(name);
  if (v == nullptr || *v == 0) return fallback;
  const long x = std::strtol(v, nullptr, 10);
  return x > 0 ? static_cast<int32_t>(x) : fallback;
}

// Split sizing: enough workgroups to cover 256 CUs several times over, each
// split a whole number of tiles, and its page list within the LDS cache.
decode_plan plan_decode(const pool_layout &L, int32_t n_seq, int32_t max_kv_len) {
  decode_plan p;
  const int32_t lpt = L.head_dim / 16;
  const int32_t tile = 2 * (k_threads / lpt);
  const int32_t units = n_seq * L.n_head_kv;
  const int32_t target = env_int("EMELK_DECODE_TARGET_WG", 2048);
  const int32_t tiles = (max_kv_len + tile - 1) / tile;
  int32_t splits = (target + units - 1) / units;
  splits = splits < 1 ? 1 : (splits > tiles ? tiles : splits);
  const int32_t forced = env_int("EMELK_DECODE_SPLITS", 0);
  if (forced > 0) splits = forced < tiles ? forced : tiles;
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

template <int D, int G, bool Q8>
void launch_decode(const decode_params &P, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((decode_kernel<D, G, Q8>), grid, dim3(k_threads), 0, st, P);
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

}  // namespace
}  // namespace emelk

extern "C" emel_error_type emelk_attn_decode_workspace_size(const emelk_kv_geometry *g,
                                                            int32_t n_seq, int32_t max_kv_len,
                                                            uint64_t *bytes_out) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || bytes_out == nullptr || n_seq <= 0 ||
      max_kv_len <= 0) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  *bytes_out = emelk::plan_decode(L, n_seq, max_kv_len).workspace_bytes;
  return EMELK_ERR_NONE;
}

extern "C" emel_error_type emelk_attn_decode(const emelk_kv_geometry *g, const void *k_pool,
                                             const void *v_pool, int32_t layer, const float *q,
                                             float *out, int32_t n_seq, const int32_t *kv_lens,
                                             int32_t max_kv_len, const uint16_t *block_tables,
                                             int32_t table_stride, float scale, void *workspace,
                                             uint64_t workspace_bytes, void *stream) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || k_pool == nullptr || v_pool == nullptr ||
      q == nullptr || out == nullptr || kv_lens == nullptr || block_tables == nullptr ||
      workspace == nullptr || layer < 0 || layer >= L.n_layer || n_seq <= 0 || n_seq > 65535 ||
      max_kv_len <= 0 || table_stride <= 0 || !(scale > 0.0f) || !std::isfinite(scale)) {
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
  const uint64_t acc_floats = static_cast<uint64_t>(n_seq) * L.n_head * plan.max_splits * L.head_dim;
  P.part_acc = static_cast<float *>(workspace);
  P.part_ml = P.part_acc + acc_floats;
  const dim3 grid(plan.max_splits, L.n_head_kv, n_seq);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int32_t group = L.n_head / L.n_head_kv;
  const bool q8 = L.kv_type == EMELK_KV_Q8_0;
  bool ok = false;
  if (L.head_dim == 128) {
    ok = q8 ? emelk::dispatch_group<128, true>(group, P, grid, st)
            : emelk::dispatch_group<128, false>(group, P, grid, st);
  } else {
    ok = q8 ? emelk::dispatch_group<64, true>(group, P, grid, st)
            : emelk::dispatch_group<64, false>(group, P, grid, st);
  }
  if (!ok) return EMELK_ERR_INVALID_REQUEST;
  const dim3 cgrid(n_seq * L.n_head);
  if (L.head_dim == 128) {
    hipLaunchKernelGGL(emelk::combine_kernel<128>, cgrid, dim3(128), 0, st, P.part_acc, P.part_ml,
                       kv_lens, L.n_head, plan.max_splits, plan.tokens_per_split, P.c, out);
  } else {
    hipLaunchKernelGGL(emelk::combine_kernel<64>, cgrid, dim3(64), 0, st, P.part_acc, P.part_ml,
                       kv_lens, L.n_head, plan.max_splits, plan.tokens_per_split, P.c, out);
  }
  return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
}
