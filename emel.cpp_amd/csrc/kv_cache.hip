// Page-pool kernels: append (f16 and on-the-fly q8_0), block-table gather and
// batched page copies (copy-on-write tail split, eviction compaction), plus
// the device KV owner object.  All are HBM-bound byte/integer work: 16-byte
// coalesced accesses, no LDS, no MFMA.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <new>

#include "device_common.hpp"
#include "emelk.h"
#include "pool_layout.hpp"
#include "q8_device.hpp"

namespace emelk {
namespace {

using namespace emelk::dev;

constexpr int k_threads = 256;

__device__ __forceinline__ bool page_ok(uint32_t page, int32_t max_blocks) {
  return page < static_cast<uint32_t>(max_blocks);
}

// ---- append, f16 --------------------------------------------------------
// One thread per 8 values of one (seq, token, kv_head) row: two 16-byte fp32
// loads, RNE conversion, one 16-byte store into the page.  Matches
// store_fp16_rounded_cache + physical_kv_position
// (text/generator/detail.hpp:2976-2982, 3050-3055).
__global__ __launch_bounds__(k_threads) void append_f16_kernel(
    pool_layout L, uint8_t *__restrict__ k_pool, uint8_t *__restrict__ v_pool, int32_t layer,
    const float *__restrict__ k_rows, const float *__restrict__ v_rows, int32_t n_seq,
    int32_t n_tokens, const int32_t *__restrict__ positions, const uint16_t *__restrict__ tables,
    int32_t table_stride) {
  const int32_t chunks = L.head_dim / 8;
  const uint64_t total = static_cast<uint64_t>(n_seq) * n_tokens * L.n_head_kv * chunks;
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(k_threads) + threadIdx.x; i < total;
       i += static_cast<uint64_t>(gridDim.x) * k_threads) {
    const int32_t c = static_cast<int32_t>(i % chunks);
    uint64_t r = i / chunks;
    const int32_t kvh = static_cast<int32_t>(r % L.n_head_kv);
    r /= L.n_head_kv;
    const int32_t t = static_cast<int32_t>(r % n_tokens);
    const int32_t s = static_cast<int32_t>(r / n_tokens);
    const int32_t pos = positions[s] + t;
    if (pos < 0) continue;
    const int32_t lb = pos / L.block_tokens;
    if (lb >= table_stride) continue;
    const uint32_t page = tables[static_cast<uint64_t>(s) * table_stride + lb];
    if (!page_ok(page, L.max_blocks)) continue;
    const int32_t off = pos % L.block_tokens;
    const uint64_t src = ((static_cast<uint64_t>(s) * n_tokens + t) * L.n_head_kv + kvh) *
                             static_cast<uint64_t>(L.head_dim) +
                         static_cast<uint64_t>(c) * 8u;
    const uint64_t dst = L.region_offset(layer, static_cast<int32_t>(page), kvh) +
                         (static_cast<uint64_t>(off) * L.head_dim + c * 8u) * 2u;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const float *rows = kv == 0 ? k_rows : v_rows;
      uint8_t *pool = kv == 0 ? k_pool : v_pool;
      const float4_t a = *reinterpret_cast<const float4_t *>(rows + src);
      const float4_t b = *reinterpret_cast<const float4_t *>(rows + src + 4);
      uint4_t out;
      out.x = as_u32(pack_half2(a.x, a.y));
      out.y = as_u32(pack_half2(a.z, a.w));
      out.z = as_u32(pack_half2(b.x, b.y));
      out.w = as_u32(pack_half2(b.z, b.w));
      store16(pool + dst, out);
    }
  }
}

// ---- append, q8_0 -------------------------------------------------------
// One thread per 32-value block (quantize_block32, q8_device.hpp).
__global__ __launch_bounds__(k_threads) void append_q8_0_kernel(
    pool_layout L, uint8_t *__restrict__ k_pool, uint8_t *__restrict__ v_pool, int32_t layer,
    const float *__restrict__ k_rows, const float *__restrict__ v_rows, int32_t n_seq,
    int32_t n_tokens, const int32_t *__restrict__ positions, const uint16_t *__restrict__ tables,
    int32_t table_stride) {
  const int32_t blocks = L.head_dim / 32;
  const uint64_t total = static_cast<uint64_t>(n_seq) * n_tokens * L.n_head_kv * blocks * 2u;
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(k_threads) + threadIdx.x; i < total;
       i += static_cast<uint64_t>(gridDim.x) * k_threads) {
    const int32_t kv = static_cast<int32_t>(i & 1u);
    uint64_t r = i >> 1;
    const int32_t blk = static_cast<int32_t>(r % blocks);
    r /= blocks;
    const int32_t kvh = static_cast<int32_t>(r % L.n_head_kv);
    r /= L.n_head_kv;
    const int32_t t = static_cast<int32_t>(r % n_tokens);
    const int32_t s = static_cast<int32_t>(r / n_tokens);
    const int32_t pos = positions[s] + t;
    if (pos < 0) continue;
    const int32_t lb = pos / L.block_tokens;
    if (lb >= table_stride) continue;
    const uint32_t page = tables[static_cast<uint64_t>(s) * table_stride + lb];
    if (!page_ok(page, L.max_blocks)) continue;
    const int32_t off = pos % L.block_tokens;
    const float *src = (kv == 0 ? k_rows : v_rows) +
                       ((static_cast<uint64_t>(s) * n_tokens + t) * L.n_head_kv + kvh) *
                           static_cast<uint64_t>(L.head_dim) +
                       static_cast<uint64_t>(blk) * 32u;
    uint8_t *region = (kv == 0 ? k_pool : v_pool) + L.region_offset(layer, static_cast<int32_t>(page), kvh);
    int8_t qs[32];
    uint16_t d;
    quantize_block32(src, qs, d);
    uint4_t *dst = reinterpret_cast<uint4_t *>(region + static_cast<uint64_t>(off) * L.head_dim +
                                               static_cast<uint64_t>(blk) * 32u);
    dst[0] = __builtin_bit_cast(uint4_t, *reinterpret_cast<int8_t(*)[16]>(qs));
    dst[1] = __builtin_bit_cast(uint4_t, *reinterpret_cast<int8_t(*)[16]>(qs + 16));
    uint16_t *scales = reinterpret_cast<uint16_t *>(region + L.scale_plane());
    scales[static_cast<uint64_t>(off) * blocks + blk] = d;
  }
}

// ---- gather -------------------------------------------------------------
// Dense head-major copy of logical tokens [0, lengths[s]) through the block
// table; positions at or past the length are written as zeros.
__global__ __launch_bounds__(k_threads) void gather_f16_kernel(
    pool_layout L, const uint8_t *__restrict__ k_pool, const uint8_t *__restrict__ v_pool,
    int32_t layer, int32_t n_seq, const int32_t *__restrict__ lengths,
    const uint16_t *__restrict__ tables, int32_t table_stride, uint8_t *__restrict__ k_out,
    uint8_t *__restrict__ v_out, int32_t out_tokens) {
  const int32_t chunks = L.head_dim / 8;
  const uint64_t total = static_cast<uint64_t>(n_seq) * L.n_head_kv * out_tokens * chunks;
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(k_threads) + threadIdx.x; i < total;
       i += static_cast<uint64_t>(gridDim.x) * k_threads) {
    const int32_t c = static_cast<int32_t>(i % chunks);
    uint64_t r = i / chunks;
    const int32_t tok = static_cast<int32_t>(r % out_tokens);
    r /= out_tokens;
    const int32_t kvh = static_cast<int32_t>(r % L.n_head_kv);
    const int32_t s = static_cast<int32_t>(r / L.n_head_kv);
    uint4_t kval = {0u, 0u, 0u, 0u};
    uint4_t vval = {0u, 0u, 0u, 0u};
    if (tok < lengths[s] && tok / L.block_tokens < table_stride) {
      const uint32_t page = tables[static_cast<uint64_t>(s) * table_stride + tok / L.block_tokens];
      if (page_ok(page, L.max_blocks)) {
        const uint64_t src = L.region_offset(layer, static_cast<int32_t>(page), kvh) +
                             (static_cast<uint64_t>(tok % L.block_tokens) * L.head_dim + c * 8u) * 2u;
        kval = load16(k_pool + src);
        vval = load16(v_pool + src);
      }
    }
    const uint64_t dst = i * 16u;
    store16(k_out + dst, kval);
    store16(v_out + dst, vval);
  }
}

// q8_0 gather emits GGUF block_q8_0 (uint16 d, int8 qs[32]; 34 bytes,
// kernel/detail.hpp:226-229): one thread per block.
__global__ __launch_bounds__(k_threads) void gather_q8_0_kernel(
    pool_layout L, const uint8_t *__restrict__ k_pool, const uint8_t *__restrict__ v_pool,
    int32_t layer, int32_t n_seq, const int32_t *__restrict__ lengths,
    const uint16_t *__restrict__ tables, int32_t table_stride, uint8_t *__restrict__ k_out,
    uint8_t *__restrict__ v_out, int32_t out_tokens) {
  const int32_t blocks = L.head_dim / 32;
  const uint64_t total = static_cast<uint64_t>(n_seq) * L.n_head_kv * out_tokens * blocks;
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(k_threads) + threadIdx.x; i < total;
       i += static_cast<uint64_t>(gridDim.x) * k_threads) {
    const int32_t blk = static_cast<int32_t>(i % blocks);
    uint64_t r = i / blocks;
    const int32_t tok = static_cast<int32_t>(r % out_tokens);
    r /= out_tokens;
    const int32_t kvh = static_cast<int32_t>(r % L.n_head_kv);
    const int32_t s = static_cast<int32_t>(r / L.n_head_kv);
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      uint16_t words[17];
#pragma unroll
      for (int w = 0; w < 17; ++w) words[w] = 0;
      if (tok < lengths[s] && tok / L.block_tokens < table_stride) {
        const uint32_t page = tables[static_cast<uint64_t>(s) * table_stride + tok / L.block_tokens];
        if (page_ok(page, L.max_blocks)) {
          const uint8_t *region = (kv == 0 ? k_pool : v_pool) +
                                  L.region_offset(layer, static_cast<int32_t>(page), kvh);
          const int32_t off = tok % L.block_tokens;
          const uint4_t *qs = reinterpret_cast<const uint4_t *>(
              region + static_cast<uint64_t>(off) * L.head_dim + static_cast<uint64_t>(blk) * 32u);
          const uint4_t q0 = qs[0];
          const uint4_t q1 = qs[1];
          words[0] = reinterpret_cast<const uint16_t *>(region + L.scale_plane())
              [static_cast<uint64_t>(off) * blocks + blk];
          const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            words[1 + 2 * w] = static_cast<uint16_t>(qw[w] & 0xFFFFu);
            words[2 + 2 * w] = static_cast<uint16_t>(qw[w] >> 16);
          }
        }
      }
      uint16_t *dst = reinterpret_cast<uint16_t *>((kv == 0 ? k_out : v_out) + i * 34u);
#pragma unroll
      for (int w = 0; w < 17; ++w) dst[w] = words[w];
    }
  }
}

// ---- batched page copy --------------------------------------------------
// One workgroup per (move, layer, K|V): a contiguous page_bytes copy with
// 16-byte accesses.
__global__ __launch_bounds__(k_threads) void copy_blocks_kernel(pool_layout L,
                                                                uint8_t *__restrict__ k_pool,
                                                                uint8_t *__restrict__ v_pool,
                                                                const int32_t *__restrict__ moves) {
  const int32_t m = blockIdx.z;
  const int32_t layer = blockIdx.y;
  uint8_t *pool = blockIdx.x == 0 ? k_pool : v_pool;
  const int32_t src = moves[2 * m];
  const int32_t dst = moves[2 * m + 1];
  if (src < 0 || dst < 0 || src >= L.max_blocks || dst >= L.max_blocks || src == dst) return;
  const uint8_t *s = pool + L.region_offset(layer, src, 0);
  uint8_t *d = pool + L.region_offset(layer, dst, 0);
  const uint64_t n16 = L.page_bytes / 16u;
  // batches of 8 loads issued before their stores keep 8 x 16 B per thread
  // in flight; the source is read once, so its loads carry the
  // non-temporal hint (measured 311 vs 337 us for the config-5 compaction,
  // 218 moves x 32 layers x K,V; non-temporal stores as well: 340 us)
  constexpr int kB = 8;
  uint64_t i = threadIdx.x;
  for (; i + (kB - 1) * k_threads < n16; i += kB * k_threads) {
    uint4_t v[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) v[b] = load16_stream(s + (i + b * k_threads) * 16u);
#pragma unroll
    for (int b = 0; b < kB; ++b) store16(d + (i + b * k_threads) * 16u, v[b]);
  }
  for (; i < n16; i += k_threads) store16(d + i * 16u, load16_stream(s + i * 16u));
}

int grid_for(uint64_t work_items) {
  const uint64_t blocks = (work_items + k_threads - 1) / k_threads;
  const uint64_t cap = 256u * 32u;  // 32 workgroups per CU on 256 CUs, grid-stride beyond
  return static_cast<int>(blocks < 1 ? 1 : (blocks > cap ? cap : blocks));
}

emel_error_type launch_status() {
  return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
}

}  // namespace
}  // namespace emelk

using emelk::pool_layout;

extern "C" emel_error_type emelk_kv_pool_bytes(const emelk_kv_geometry *g, uint64_t *bytes_out) {
  pool_layout L;
  const emel_error_type e = emelk::make_pool_layout(g, L);
  if (e != EMELK_ERR_NONE || bytes_out == nullptr) return e | (bytes_out ? 0u : EMELK_ERR_INVALID_REQUEST);
  *bytes_out = L.pool_bytes;
  return EMELK_ERR_NONE;
}

extern "C" emel_error_type emelk_kv_append(const emelk_kv_geometry *g, void *k_pool, void *v_pool,
                                           int32_t layer, const float *k_rows,
                                           const float *v_rows, int32_t n_seq, int32_t n_tokens,
                                           const int32_t *positions, const uint16_t *block_tables,
                                           int32_t table_stride, void *stream) {
  pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || k_pool == nullptr || v_pool == nullptr ||
      k_rows == nullptr || v_rows == nullptr || positions == nullptr || block_tables == nullptr ||
      layer < 0 || layer >= L.n_layer || n_seq < 0 || n_tokens < 0 || table_stride <= 0) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  if (n_seq == 0 || n_tokens == 0) return EMELK_ERR_NONE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t rows = static_cast<uint64_t>(n_seq) * n_tokens * L.n_head_kv;
  if (L.kv_type == EMELK_KV_F16) {
    hipLaunchKernelGGL(emelk::append_f16_kernel, dim3(emelk::grid_for(rows * (L.head_dim / 8))),
                       dim3(emelk::k_threads), 0, st, L, static_cast<uint8_t *>(k_pool),
                       static_cast<uint8_t *>(v_pool), layer, k_rows, v_rows, n_seq, n_tokens,
                       positions, block_tables, table_stride);
  } else {
    hipLaunchKernelGGL(emelk::append_q8_0_kernel,
                       dim3(emelk::grid_for(rows * (L.head_dim / 32) * 2u)), dim3(emelk::k_threads),
                       0, st, L, static_cast<uint8_t *>(k_pool), static_cast<uint8_t *>(v_pool),
                       layer, k_rows, v_rows, n_seq, n_tokens, positions, block_tables,
                       table_stride);
  }
  return emelk::launch_status();
}

extern "C" emel_error_type emelk_kv_gather(const emelk_kv_geometry *g, const void *k_pool,
                                           const void *v_pool, int32_t layer, int32_t n_seq,
                                           const int32_t *lengths, const uint16_t *block_tables,
                                           int32_t table_stride, void *k_out, void *v_out,
                                           int32_t out_tokens, void *stream) {
  pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || k_pool == nullptr || v_pool == nullptr ||
      lengths == nullptr || block_tables == nullptr || k_out == nullptr || v_out == nullptr ||
      layer < 0 || layer >= L.n_layer || n_seq < 0 || out_tokens < 0 || table_stride <= 0) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  if (n_seq == 0 || out_tokens == 0) return EMELK_ERR_NONE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t rows = static_cast<uint64_t>(n_seq) * L.n_head_kv * out_tokens;
  if (L.kv_type == EMELK_KV_F16) {
    hipLaunchKernelGGL(emelk::gather_f16_kernel, dim3(emelk::grid_for(rows * (L.head_dim / 8))),
                       dim3(emelk::k_threads), 0, st, L, static_cast<const uint8_t *>(k_pool),
                       static_cast<const uint8_t *>(v_pool), layer, n_seq, lengths, block_tables,
                       table_stride, static_cast<uint8_t *>(k_out), static_cast<uint8_t *>(v_out),
                       out_tokens);
  } else {
    hipLaunchKernelGGL(emelk::gather_q8_0_kernel, dim3(emelk::grid_for(rows * (L.head_dim / 32))),
                       dim3(emelk::k_threads), 0, st, L, static_cast<const uint8_t *>(k_pool),
                       static_cast<const uint8_t *>(v_pool), layer, n_seq, lengths, block_tables,
                       table_stride, static_cast<uint8_t *>(k_out), static_cast<uint8_t *>(v_out),
                       out_tokens);
  }
  return emelk::launch_status();
}

extern "C" emel_error_type emelk_kv_copy_blocks(const emelk_kv_geometry *g, void *k_pool,
                                                void *v_pool, const int32_t *moves,
                                                int32_t n_moves, void *stream) {
  pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || k_pool == nullptr || v_pool == nullptr ||
      n_moves < 0 || (n_moves > 0 && moves == nullptr) || n_moves > 65535) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  if (n_moves == 0) return EMELK_ERR_NONE;
  hipLaunchKernelGGL(emelk::copy_blocks_kernel, dim3(2, L.n_layer, n_moves), dim3(emelk::k_threads),
                     0, static_cast<hipStream_t>(stream), L, static_cast<uint8_t *>(k_pool),
                     static_cast<uint8_t *>(v_pool), moves);
  return emelk::launch_status();
}

// ---- device KV owner ------------------------------------------------------
struct emelk_kv_cache {
  emelk_kv_geometry geometry;
  pool_layout layout;
  void *k_pool = nullptr;
  void *v_pool = nullptr;
  int32_t *move_slot = nullptr;  // device int32[2] for single-page copies
  int32_t *move_host = nullptr;  // pinned staging for move_slot
  hipStream_t stream = nullptr;
  // device view upload: pinned snapshot staging (allocated on first use)
  // and the event that tells when the previous upload has read it
  emelk_view_snapshot *view_host = nullptr;
  hipEvent_t view_read = nullptr;
  bool view_pending = false;
};

extern "C" emel_error_type emelk_kv_cache_create(const emelk_kv_geometry *g, void *stream,
                                                 emelk_kv_cache **cache_out) {
  if (cache_out == nullptr) return EMELK_ERR_INVALID_REQUEST;
  *cache_out = nullptr;
  pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE) return EMELK_ERR_INVALID_REQUEST;
  auto *c = new (std::nothrow) emelk_kv_cache();
  if (c == nullptr) return EMELK_ERR_OUT_OF_MEMORY;
  c->geometry = *g;
  c->layout = L;
  c->stream = static_cast<hipStream_t>(stream);
  if (hipMalloc(&c->k_pool, L.pool_bytes) != hipSuccess ||
      hipMalloc(&c->v_pool, L.pool_bytes) != hipSuccess ||
      hipMalloc(reinterpret_cast<void **>(&c->move_slot), 2 * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc(reinterpret_cast<void **>(&c->move_host), 2 * sizeof(int32_t),
                    hipHostMallocDefault) != hipSuccess) {
    emelk_kv_cache_destroy(c);
    return EMELK_ERR_OUT_OF_MEMORY;
  }
  *cache_out = c;
  return EMELK_ERR_NONE;
}

extern "C" void emelk_kv_cache_destroy(emelk_kv_cache *c) {
  if (c == nullptr) return;
  if (c->stream != nullptr) (void)hipStreamSynchronize(c->stream);
  else (void)hipDeviceSynchronize();
  if (c->k_pool) (void)hipFree(c->k_pool);
  if (c->v_pool) (void)hipFree(c->v_pool);
  if (c->move_slot) (void)hipFree(c->move_slot);
  if (c->move_host) (void)hipHostFree(c->move_host);
  if (c->view_host) (void)hipHostFree(c->view_host);
  if (c->view_read) (void)hipEventDestroy(c->view_read);
  delete c;
}

// capture_view (kv/sm.hpp:448-465 -> view::snapshot, memory/view.hpp:59-117)
// delivered to device memory: the actor fills the pinned staging snapshot,
// which is copied on the cache's stream, so the copy is ordered with the
// page copies of earlier allocate_slots calls and before later kernels.
extern "C" emel_error_type emelk_kv_cache_upload_view(emelk_kv_cache *c, emelk_kv_actor *actor,
                                                      emelk_view_snapshot *view_dev) {
  if (c == nullptr || actor == nullptr || view_dev == nullptr) return EMELK_ERR_INVALID_REQUEST;
  if (c->view_host == nullptr) {
    if (hipHostMalloc(reinterpret_cast<void **>(&c->view_host), sizeof(emelk_view_snapshot),
                      hipHostMallocDefault) != hipSuccess) {
      c->view_host = nullptr;
      return EMELK_ERR_OUT_OF_MEMORY;
    }
    if (hipEventCreateWithFlags(&c->view_read, hipEventDisableTiming) != hipSuccess) {
      c->view_read = nullptr;
      return EMELK_ERR_BACKEND;
    }
  }
  if (c->view_pending) {  // the copy engine may still read the staging snapshot
    if (hipEventSynchronize(c->view_read) != hipSuccess) return EMELK_ERR_BACKEND;
    c->view_pending = false;
  }
  int32_t err = EMELK_ERR_NONE;
  emelk_event_capture_view ev{c->view_host, &err};
  if (!emelk_kv_capture_view(actor, &ev)) {
    return err != EMELK_ERR_NONE ? static_cast<emel_error_type>(err) : EMELK_ERR_INTERNAL;
  }
  if (hipMemcpyAsync(view_dev, c->view_host, sizeof(emelk_view_snapshot), hipMemcpyHostToDevice,
                     c->stream) != hipSuccess ||
      hipEventRecord(c->view_read, c->stream) != hipSuccess) {
    return EMELK_ERR_BACKEND;
  }
  c->view_pending = true;
  return EMELK_ERR_NONE;
}

extern "C" void *emelk_kv_cache_k_pool(emelk_kv_cache *c) { return c ? c->k_pool : nullptr; }
extern "C" void *emelk_kv_cache_v_pool(emelk_kv_cache *c) { return c ? c->v_pool : nullptr; }
extern "C" void *emelk_kv_cache_stream(const emelk_kv_cache *c) {
  return c ? static_cast<void *>(c->stream) : nullptr;
}

// allocate_slots::copy_block_fn target (text/generator/context.hpp:36-50 ->
// copy_attention_kv_block, detail.hpp:3334-3417): validates the request like
// the reference (block_tokens must match the pool, ids in range), then
// enqueues one page move.  The staging buffer is reused, so the call waits
// for the previous single-page copy's upload before overwriting it.
extern "C" bool emelk_kv_cache_copy_block(int32_t src_block, int32_t dst_block,
                                          int32_t block_tokens, void *user_data,
                                          int32_t *error_out) {
  auto *c = static_cast<emelk_kv_cache *>(user_data);
  if (error_out) *error_out = EMELK_ERR_NONE;
  if (c == nullptr || block_tokens != c->layout.block_tokens || src_block < 0 || dst_block < 0 ||
      src_block >= c->layout.max_blocks || dst_block >= c->layout.max_blocks) {
    if (error_out) *error_out = EMELK_ERR_INVALID_REQUEST;
    return false;
  }
  if (hipStreamSynchronize(c->stream) != hipSuccess) {
    if (error_out) *error_out = EMELK_ERR_BACKEND;
    return false;
  }
  c->move_host[0] = src_block;
  c->move_host[1] = dst_block;
  if (hipMemcpyAsync(c->move_slot, c->move_host, 2 * sizeof(int32_t), hipMemcpyHostToDevice,
                     c->stream) != hipSuccess ||
      emelk_kv_copy_blocks(&c->geometry, c->k_pool, c->v_pool, c->move_slot, 1, c->stream) !=
          EMELK_ERR_NONE) {
    if (error_out) *error_out = EMELK_ERR_BACKEND;
    return false;
  }
  return true;
}
