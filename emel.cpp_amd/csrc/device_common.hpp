// Shared device helpers for the gfx950 kernels (wave64, CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emelk::dev {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef int32_t int4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

constexpr int k_wave = 64;

// RNE fp32 -> f16 (v_cvt_f16_f32 under the default round-to-nearest-even mode).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  const half_t h = static_cast<half_t>(v);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(half_t, b));
}

__device__ __forceinline__ half2_t as_half2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Packs two fp32 values into a half2 with RNE rounding.
__device__ __forceinline__ half2_t pack_half2(float lo, float hi) {
  half2_t r;
  r.x = static_cast<half_t>(lo);
  r.y = static_cast<half_t>(hi);
  return r;
}

// fp32 += a.x*b.x + a.y*b.y  (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c) {
  return __builtin_amdgcn_fdot2(a, b, c, false);
}

// DPP cross-lane moves inside 16-lane rows (gfx9 encodings).
// All controls used here read a valid lane for every lane, so no "old"
// value is needed (mov_dpp), which lets the compiler fold the move into the
// consuming v_add_f32_dpp.
template <int ctrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, true));
}
constexpr int k_dpp_quad_xor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int k_dpp_quad_xor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int k_dpp_row_half_mirror = 0x141;
constexpr int k_dpp_row_mirror = 0x140;

// Sum over aligned groups of `lanes` consecutive lanes (lanes in
// {2,4,8,16,32}); every lane of the group receives the group total.
template <int lanes>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(lanes == 2 || lanes == 4 || lanes == 8 || lanes == 16 || lanes == 32,
                "group size");
  v += dpp<k_dpp_quad_xor1>(v);
  if constexpr (lanes >= 4) v += dpp<k_dpp_quad_xor2>(v);
  if constexpr (lanes >= 8) v += dpp<k_dpp_row_half_mirror>(v);
  if constexpr (lanes >= 16) v += dpp<k_dpp_row_mirror>(v);
  if constexpr (lanes >= 32) v += __shfl_xor(v, 16, 64);  // the neighbouring 16-lane row
  return v;
}

constexpr int k_dpp_row_ror4 = 0x124;
constexpr int k_dpp_row_ror8 = 0x128;

// v + (v of the lane `bit` lanes away) for bit 16 or 32, by the gfx950
// row-swap permutes: with both operands v, the two results are v and its
// partner in some order, so every lane of the pair gets the same sum.
template <int bit>
__device__ __forceinline__ float pair_sum_rows(float v) {
  static_assert(bit == 16 || bit == 32, "row pair");
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  if constexpr (bit == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
           __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
           __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
  }
}

// Value of lane `src` of each aligned group of 4 lanes (DPP quad_perm).
template <int src>
__device__ __forceinline__ float quad_bcast(float v) {
  return dpp<src | (src << 2) | (src << 4) | (src << 6)>(v);
}

// Sum over the `chunks` lanes that differ only in lane bits 2 .. 2 +
// log2(chunks) - 1 (chunks in {4, 8, 16}); every lane receives the total.
template <int chunks>
__device__ __forceinline__ float chunk_sum(float v) {
  static_assert(chunks == 4 || chunks == 8 || chunks == 16, "chunk count");
  v += dpp<k_dpp_row_ror8>(v);  // lane bit 3 (rotation by 8 in a 16-lane row)
  v += dpp<k_dpp_row_ror4>(v);  // bit 2: v is already symmetric in bit 3
  if constexpr (chunks >= 8) v = pair_sum_rows<16>(v);
  if constexpr (chunks >= 16) v = pair_sum_rows<32>(v);
  return v;
}

__device__ __forceinline__ float wave_shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, k_wave);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16-byte streaming load: non-temporal hint, for data read once (K/V rows
// in decode); measured on MI355X it lifts sustained HBM reads from ~6.3 to
// ~7.1 TB/s versus plain loads.
__device__ __forceinline__ uint4_t load16_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(p));
}
__device__ __forceinline__ uint2_t load8_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint2_t *>(p));
}
__device__ __forceinline__ uint32_t load4_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ uint32_t load2_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}

// 16-byte global load/store.
__device__ __forceinline__ uint4_t load16(const void *p) {
  return *reinterpret_cast<const uint4_t *>(p);
}
__device__ __forceinline__ void store16(void *p, uint4_t v) {
  *reinterpret_cast<uint4_t *>(p) = v;
}

}  // namespace emelk::dev
