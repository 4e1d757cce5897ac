// Chunked-prefill attention on MFMA (gfx950 v_mfma_f32_32x32x16_f16).
//
// Replaces the reference's per-row chunked prefill (run_prefill's store +
// attend loop, text/generator/detail.hpp:4297-4372: row r of the chunk
// attends causally to logical positions [0, q_start + r]) with one flash
// attention pass per chunk.
//
// Workgroup = 4 waves = one KV head, G_WG query heads of its group and RB
// row blocks of 32 query rows (G_WG * RB = 4), so the four waves share every
// K/V tile staged in LDS.  Per 32-key tile each wave computes
//     S^T (32 keys x 32 rows)  = K (32 x D) . Q^T (D x 32)      D/16 MFMAs
// so a lane holds 16 of the 32 scores of ONE query row (the other 16 sit in
// the lane 32 apart): the row max and sum are in-lane plus one cross-half
// swap.  The fp32 score accumulator converted to fp16 is directly the A
// operand of
//     O (32 rows x D) += P (32 x 32 keys) . V (32 x D)        2*D/32 MFMAs
// provided the keys of V are staged in LDS in the order the accumulator
// holds them (sigma below), which the staging does while transposing V.
// Online softmax in fp32 (exp2 with the scale folded in); Q is rounded to
// fp16 as round_q_for_nonflash does (detail.hpp:2898-2903) and P is fp16,
// as the reference's rounded probabilities are (detail.hpp:3146-3149).
// K/V tiles are double-buffered: the next tile's global loads are issued
// before the current tile's MFMAs.
#include <hip/hip_runtime.h>

#include <cmath>

#include "device_common.hpp"
#include "emelk.h"
#include "pool_layout.hpp"

namespace emelk {
namespace {

using namespace emelk::dev;

constexpr int k_threads = 256;
constexpr int k_tile = 32;  // keys per tile

typedef _Float16 half8_v __attribute__((ext_vector_type(8)));
typedef float float16_v __attribute__((ext_vector_type(16)));

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
};

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

template <int D, int G_WG, int RB>
__global__ __launch_bounds__(k_threads) void prefill_kernel(prefill_params P) {
  static_assert(G_WG * RB == 4, "four waves per workgroup");
  constexpr int KSTEPS = D / 16;   // MFMA k-steps for S^T
  constexpr int DCH = D / 32;      // 32-wide dim chunks of O
  constexpr int KROW = D + 8;      // padded LDS row (halves) of K
  constexpr int VROW = k_tile + 8; // padded LDS row (halves) of V^T
  constexpr int PARTS = k_threads / k_tile;  // staging threads per key row (8)
  constexpr int PW = D / PARTS;              // dims per staging thread (16 or 8)
  constexpr int NL = PW / 8;                 // 16-byte loads per row part

  __shared__ half_t s_k[2][k_tile][KROW];
  __shared__ half_t s_vt[2][D][VROW];
  __shared__ float s_row[4][32];

  const int tid = threadIdx.x;
  const int wave = tid / k_wave;
  const int lane = tid % k_wave;
  const int h = lane / 32;
  const int l32 = lane % 32;
  const int seq = blockIdx.z;
  const int group = P.L.n_head / P.L.n_head_kv;
  const int head0 = blockIdx.y * G_WG;
  const int kvh = head0 / group;
  const int head = head0 + wave % G_WG;
  const int row0 = (blockIdx.x * RB + wave / G_WG) * 32;
  const int n_q = P.n_q;
  const int q0 = P.q_start[seq];
  const int total = q0 + n_q;
  const int wg_row_end = min(n_q, (blockIdx.x + 1) * RB * 32);
  if (blockIdx.x * RB * 32 >= n_q) return;
  const int key_end = q0 + wg_row_end;  // exclusive
  const int n_tiles = (key_end + k_tile - 1) / k_tile;
  const int my_row = row0 + l32;
  const bool row_ok = my_row < n_q;
  const int my_pos = q0 + my_row;

  // Q^T operand (B): lane holds query my_row, dims 16*kk + 8*h .. +7.
  half8_v qop[KSTEPS];
  {
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

  float16_v o[DCH];
#pragma unroll
  for (int c = 0; c < DCH; ++c) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[c][r] = 0.0f;
  }
  float m = -INFINITY;
  float l = 0.0f;

  // staging: thread -> (key, PW-dim part) of the 32-key tile
  const int st_part = tid % PARTS;
  const int st_key = tid / PARTS;
  const uint64_t layer_base = static_cast<uint64_t>(P.layer) * P.L.layer_bytes +
                              static_cast<uint64_t>(kvh) * P.L.region_bytes;
  const uint16_t *table = P.tables + static_cast<uint64_t>(seq) * P.table_stride;
  uint4_t rk[2], rv[2];

  auto load_tile = [&](int t) {
    const int key = t * k_tile + st_key;
    const int lb = key / P.L.block_tokens;
    uint32_t page = 0xFFFFFFFFu;
    if (key < total && lb < P.table_stride) page = table[lb];
#pragma unroll
    for (int j = 0; j < 2; ++j) rk[j] = rv[j] = uint4_t{0u, 0u, 0u, 0u};
    if (page < static_cast<uint32_t>(P.L.max_blocks)) {
      const uint64_t off = layer_base + static_cast<uint64_t>(page) * P.L.page_bytes +
                           (static_cast<uint64_t>(key % P.L.block_tokens) * D + st_part * PW) * 2u;
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        rk[j] = load16(P.k_pool + off + 16 * j);
        rv[j] = load16(P.v_pool + off + 16 * j);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      *reinterpret_cast<uint4_t *>(&s_k[buf][st_key][st_part * PW + 8 * j]) = rk[j];
    }
    const int slot = key_slot(st_key);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t w[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int dim = st_part * PW + 8 * j + 2 * e;
        s_vt[buf][dim][slot] = __builtin_bit_cast(half_t, static_cast<uint16_t>(w[e] & 0xFFFFu));
        s_vt[buf][dim + 1][slot] = __builtin_bit_cast(half_t, static_cast<uint16_t>(w[e] >> 16));
      }
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < n_tiles;
    if (more) load_tile(t + 1);

    // S^T = K . Q^T
    float16_v s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const half8_v a = *reinterpret_cast<const half8_v *>(&s_k[buf][l32][16 * kk + 8 * h]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qop[kk], s, 0, 0, 0);
    }

    // mask + online softmax for query my_row (in-lane 16 keys + other half)
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t * k_tile + 8 * (r / 4) + 4 * h + (r % 4);
      const bool ok = row_ok && key <= my_pos && key < total;
      s[r] = ok ? s[r] * P.c : -INFINITY;
      tmax = fmaxf(tmax, s[r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, k_wave));
    const float mn = fmaxf(m, tmax);
    const float ms = mn == -INFINITY ? 0.0f : mn;
    const float alpha = fast_exp2(m - ms);
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = fast_exp2(s[r] - ms);
      psum += s[r];
    }
    psum += __shfl_xor(psum, 32, k_wave);
    l = l * alpha + psum;
    m = mn;

    // alpha of each O row: rows 8a + 4h + b live in lane (row), so pass them
    // through LDS (wave-private slice)
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
#pragma unroll
    for (int c = 0; c < DCH; ++c) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[c][r] *= arow[r];
    }

    // O += P . V
    half8_v pa[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int i = 0; i < 8; ++i) pa[st][i] = static_cast<half_t>(s[8 * st + i]);
    }
#pragma unroll
    for (int c = 0; c < DCH; ++c) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const half8_v b = *reinterpret_cast<const half8_v *>(&s_vt[buf][32 * c + l32][16 * st + 8 * h]);
        o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[st], b, o[c], 0, 0, 0);
      }
    }

    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  // normalise by l of each row and write rows < n_q
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

template <int D>
bool launch_prefill(const prefill_params &P, int32_t n_seq, hipStream_t st) {
  const int group = P.L.n_head / P.L.n_head_kv;
  const int g_wg = group < 4 ? group : 4;
  const int rb = 4 / g_wg;
  const dim3 grid((P.n_q + 32 * rb - 1) / (32 * rb), P.L.n_head / g_wg, n_seq);
  switch (g_wg) {
    case 1: hipLaunchKernelGGL((prefill_kernel<D, 1, 4>), grid, dim3(k_threads), 0, st, P); return true;
    case 2: hipLaunchKernelGGL((prefill_kernel<D, 2, 2>), grid, dim3(k_threads), 0, st, P); return true;
    case 4: hipLaunchKernelGGL((prefill_kernel<D, 4, 1>), grid, dim3(k_threads), 0, st, P); return true;
    default: return false;
  }
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
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || L.kv_type != EMELK_KV_F16 ||
      k_pool == nullptr || v_pool == nullptr || q == nullptr || out == nullptr ||
      q_start == nullptr || block_tables == nullptr || layer < 0 || layer >= L.n_layer ||
      n_seq <= 0 || n_seq > 65535 || n_q <= 0 || table_stride <= 0 || !(scale > 0.0f) ||
      !std::isfinite(scale)) {
    return EMELK_ERR_INVALID_REQUEST;
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = L.head_dim == 128 ? emelk::launch_prefill<128>(P, n_seq, st)
                                    : emelk::launch_prefill<64>(P, n_seq, st);
  if (!ok) return EMELK_ERR_INVALID_REQUEST;
  return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
}
