// common.h -- shared device helpers for the gfx950 W4A8 / W4A16 decode GEMV library.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, DPP cross-lane
// moves, v_dot4_i32_i8 / v_dot2_f32_f16 dot instructions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nve_kernels.h"

namespace nve {

constexpr int kWave = 64;
constexpr int kBlock = 32;  // Q4_0 / Q8 group size (weights and activations)

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));

// ---- wavefront reductions (DPP; the total lands in lane 63) ----------------
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror, then
// row_bcast:15 into rows 1/3 and row_bcast:31 into rows 2/3.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_mov_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, false);
}

// Sum over all 64 lanes; result valid in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_mov<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);       // row_half_mirror
  v += dpp_mov<0x140>(v);       // row_mirror
  v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15 -> rows 1,3
  v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31 -> rows 2,3
  return v;
}

// Sum over all 64 lanes, broadcast to every lane.
__device__ __forceinline__ float wave_sum(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_to_lane63(v)), 63));
}

// Reductions within aligned groups of 4 lanes (all 4 lanes get the result).
__device__ __forceinline__ int quad_sum_i(int v) {
  v += dpp_mov_i<0xB1>(v);
  v += dpp_mov_i<0x4E>(v);
  return v;
}
__device__ __forceinline__ float quad_max_f(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  return v;
}
// Butterfly across the two 16-lane rows of each 32-lane half (lane l <-> l ^ 16) and
// across the two halves (l <-> l ^ 32), via v_permlane16_swap / v_permlane32_swap:
// swapping a value with itself leaves the partner's copy in one of the two results.
__device__ __forceinline__ float xor16_partner_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ float xor32_partner_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ float xor16_partner_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float xor32_partner_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}

// f64 lane moves: the two halves travel separately through the same DPP / permlane
// path.  Every step adds a lane's value to its partner's, and IEEE addition is
// commutative, so both lanes of a pair (and in the end every lane) hold the same bits.
template <int CTRL>
__device__ __forceinline__ double dpp_mov_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
template <bool X32>
__device__ __forceinline__ double xor_partner_sum_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
  const auto rl = X32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                      : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto rh = X32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                      : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  const double a = __builtin_bit_cast(double, ((uint64_t)(uint32_t)rh[0] << 32) | (uint32_t)rl[0]);
  const double b = __builtin_bit_cast(double, ((uint64_t)(uint32_t)rh[1] << 32) | (uint32_t)rl[1]);
  return a + b;
}
// f64 sum over aligned groups of N lanes, in every lane of the group (the order of
// group_sum below).
template <int N>
__device__ __forceinline__ double group_sum_f64(double v) {
  static_assert(N == 16 || N == 64, "group size");
  v += dpp_mov_f64<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov_f64<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov_f64<0x141>(v);  // row_half_mirror
  v += dpp_mov_f64<0x140>(v);  // row_mirror
  if (N >= 64) {
    v = xor_partner_sum_f64<false>(v);
    v = xor_partner_sum_f64<true>(v);
  }
  return v;
}

// Sum over aligned groups of N lanes (N = 8, 16, 32 or 64), result in every lane of
// the group: quad butterflies, then the half-row and row mirrors (a mirror maps one
// half of the group onto the other), then the permlane swaps.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 8 || N == 16 || N == 32 || N == 64, "group size");
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  if (N >= 16) v += dpp_mov<0x140>(v);  // row_mirror
  if (N >= 32) v = xor16_partner_sum(v);
  if (N >= 64) v = xor32_partner_sum(v);
  return v;
}

// Sum / max over the lanes l, l ^ S, l ^ 2S, ... (S = 8, 16 or 32): lanes holding the
// same position within their S-lane group.
template <int S>
__device__ __forceinline__ float stride_sum(float v) {
  static_assert(S == 8 || S == 16 || S == 32, "stride");
  if (S <= 8) v += dpp_mov<0x128>(v);  // row_ror:8 (lane i <- lane i-8 within its row)
  if (S <= 16) v = xor16_partner_sum(v);
  return xor32_partner_sum(v);
}
template <int S>
__device__ __forceinline__ float stride_max(float v) {
  static_assert(S == 8 || S == 16 || S == 32, "stride");
  if (S <= 8) v = fmaxf(v, dpp_mov<0x128>(v));
  if (S <= 16) v = xor16_partner_max(v);
  return xor32_partner_max(v);
}

// 4x4 transpose between the four 16-lane groups and four registers: (lane group g,
// register c) -> (lane group c, register g), via two permlane32 and two permlane16 swaps.
__device__ __forceinline__ void transpose4(uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3) {
  auto s02 = __builtin_amdgcn_permlane32_swap(c0, c2, false, false);
  auto s13 = __builtin_amdgcn_permlane32_swap(c1, c3, false, false);
  c0 = s02[0];
  c2 = s02[1];
  c1 = s13[0];
  c3 = s13[1];
  auto s01 = __builtin_amdgcn_permlane16_swap(c0, c1, false, false);
  auto s23 = __builtin_amdgcn_permlane16_swap(c2, c3, false, false);
  c0 = s01[0];
  c1 = s01[1];
  c2 = s23[0];
  c3 = s23[1];
}

// Value of v in lane src_lane (ds_bpermute: through the LDS crossbar, no LDS storage).
__device__ __forceinline__ uint32_t lane_fetch(uint32_t v, int src_lane) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane << 2, (int)v);
}
__device__ __forceinline__ uint4 lane_fetch4(uint4 v, int src_lane) {
  return make_uint4(lane_fetch(v.x, src_lane), lane_fetch(v.y, src_lane), lane_fetch(v.z, src_lane),
                    lane_fetch(v.w, src_lane));
}

// Pairs of lanes (2i, 2i+1).
__device__ __forceinline__ int pair_sum_i(int v) { return v + dpp_mov_i<0xB1>(v); }

// ---- streaming loads ----------------------------------------------------------
// Weights are read exactly once per GEMV: load them with the nontemporal hint (nt),
// which keeps the streamed bytes from displacing reusable lines in L2 / MALL.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float ld_stream(const float* p) { return __builtin_nontemporal_load(p); }

// ---- scalar conversions -----------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __builtin_bit_cast(float, h << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t x = __builtin_bit_cast(uint32_t, f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int DT>
__device__ __forceinline__ float load_act(const void* p, size_t i);
template <>
__device__ __forceinline__ float load_act<NVE_DT_F16>(const void* p, size_t i) {
  return (float)((const _Float16*)p)[i];
}
template <>
__device__ __forceinline__ float load_act<NVE_DT_BF16>(const void* p, size_t i) {
  return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
template <>
__device__ __forceinline__ float load_act<NVE_DT_F32>(const void* p, size_t i) {
  return ((const float*)p)[i];
}

template <int DT>
__device__ __forceinline__ void store_out(void* p, size_t i, float v);
// f32 -> f16, round to nearest even, of a value that is first materialised as f32:
// without the barrier the compiler may fuse the producing multiply with the
// conversion (v_fma_mix), rounding the exact product once instead of twice.
__device__ __forceinline__ _Float16 f32_to_f16_rne(float v) {
  asm volatile("" : "+v"(v));
  return (_Float16)v;
}
template <>
__device__ __forceinline__ void store_out<NVE_DT_F16>(void* p, size_t i, float v) {
  ((_Float16*)p)[i] = f32_to_f16_rne(v);
}
template <>
__device__ __forceinline__ void store_out<NVE_DT_BF16>(void* p, size_t i, float v) {
  ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}
template <>
__device__ __forceinline__ void store_out<NVE_DT_F32>(void* p, size_t i, float v) {
  ((float*)p)[i] = v;
}
template <>
__device__ __forceinline__ void store_out<NVE_DT_F32_ACCUM>(void* p, size_t i, float v) {
  ((float*)p)[i] += v;  // one writer per row
}

// Barrier that waits only for this wave's LDS traffic (not for outstanding global
// loads), so weight loads issued before it stay in flight across the barrier.
// The fences are scoped to the LDS address space ("local"), so the compiler emits
// lgkmcnt(0) before s_barrier instead of vmcnt(0).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// int8 quantization of one value already multiplied by 1/scale: round half to even,
// NaN -> 0, clamp to [-127, 127] (_nve_quantize_f16_q8, cuda/nve_kernels.cu:712-745).
__device__ __forceinline__ int8_t q8_round_clamp(float v) {
  float r = rintf(v);
  if (r != r) r = 0.0f;  // NaN -> 0
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int8_t)(int)r;
}

// Group-32 int8 quantization of 4 consecutive values per lane, 8 consecutive lanes per
// group (all 8 lanes of a group must be active): scale = absmax / 127 (1 for an
// all-zero group), codes = q8_round_clamp(v / scale); element i0 is the lane's first.
__device__ __forceinline__ void q8_group8_store(const float v[4], bool ok, int8_t* __restrict__ xq,
                                                float* __restrict__ xs, size_t i0) {
  float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  m = quad_max_f(m);
  m = fmaxf(m, dpp_mov<0x141>(m));  // row_half_mirror: the other quad of the 8 lanes
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  if (ok) {
    char4 q;
    q.x = q8_round_clamp(v[0] * inv);
    q.y = q8_round_clamp(v[1] * inv);
    q.z = q8_round_clamp(v[2] * inv);
    q.w = q8_round_clamp(v[3] * inv);
    *(char4*)(xq + i0) = q;
    if ((i0 & 31) == 0) xs[i0 >> 5] = scale;
  }
}

}  // namespace nve

// ---- host-side helpers shared by the translation units -----------------------
namespace nve_host {
int set_status(int st);  // records the last status, returns st
inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }
int launch_status();  // hipGetLastError mapped to an NVE status
}  // namespace nve_host
