// SPDX-License-Identifier: Apache-2.0
// Shared device/host helpers for the gfx950 StripedHyena2 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "ops.hpp"
#include "status.hpp"

namespace evo::hip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

// ---- BF16 helpers (raw 16-bit storage; round to nearest even).
__host__ __device__ inline float bf16_to_f32(const uint16_t bits) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16U);
}

__host__ __device__ inline uint16_t f32_to_bf16(const float value) {
#if defined(__HIP_DEVICE_COMPILE__)
  // gfx950 converts in hardware (v_cvt_pk_bf16_f32, round to nearest even).
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(value));
#endif
  const uint32_t bits = __builtin_bit_cast(uint32_t, value);
  if ((bits & 0x7fffffffU) > 0x7f800000U)
    return static_cast<uint16_t>((bits >> 16U) | 0x40U);
  return static_cast<uint16_t>((bits + 0x7fffU + ((bits >> 16U) & 1U)) >> 16U);
}

__host__ __device__ inline float round_bf16(const float value) {
  return bf16_to_f32(f32_to_bf16(value));
}

// ---- Global -> LDS DMA (global_load_lds_dwordx4): lane l's 16 bytes land at
// LDS byte address lds + 16 l (lds must be wave-uniform). Issued through
// inline asm so the compiler does not serialise it with LDS reads of other
// stage buffers (it cannot tell them apart and would wait for every DMA);
// kernels account for completion themselves with s_waitcnt vmcnt. M0 is
// written here and is not live across this asm in the kernels that use it.
typedef __attribute__((address_space(3))) void lds_void;

__device__ inline void dma16(const void *global, const void *lds) {
  const unsigned address = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<size_t>((const lds_void *)(lds))));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(global), "s"(address) : "memory");
}

// The same DMA with a wave-uniform base address (SGPR pair) and a 32-bit
// per-lane byte offset: no per-lane 64-bit address arithmetic.
__device__ inline void dma16(const void *base, uint32_t offset, const void *lds) {
  const unsigned address = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<size_t>((const lds_void *)(lds))));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(offset), "s"(base), "s"(address) : "memory");
}

template <int kPending>
__device__ inline void wait_dma() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kPending) : "memory");
}

// ---- GEMM tile order.
// Linear tile of hardware block `id` among `total` blocks: consecutive ids
// go to different XCDs, so id -> (xcd, slot) -> contiguous band per XCD.
// XCD x receives total/8 tiles (+1 for the first total%8 XCDs), so the map
// from hardware id to linear tile is a bijection for every grid size.
__device__ inline int xcd_linear(int id, int total) {
  const int q = total / 8, r = total % 8;
  const int xcd = id % 8;
  return xcd * q + min(xcd, r) + id / 8;
}

// Linear tile -> (tile_m, tile_n): groups of kGroupRows tile rows, walked
// column by column.
template <int kGroupRows = 8>
__device__ inline void tile_of_linear(int linear, int tiles_m, int tiles_n, int *tm, int *tn) {
  const int group_size = kGroupRows * tiles_n;
  const int group = linear / group_size;
  const int first_m = group * kGroupRows;
  const int rows = min(tiles_m - first_m, kGroupRows);
  const int in_group = linear % group_size;
  *tm = first_m + in_group % rows;
  *tn = in_group / rows;
}

// Hardware block id -> (tile_m, tile_n) over the whole tile grid.
template <int kGroupRows = 8>
__device__ inline void tile_of(int id, int tiles_m, int tiles_n, int *tm, int *tn) {
  tile_of_linear<kGroupRows>(xcd_linear(id, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
}

// ---- E4M3FN encoder: round to nearest even, saturating finite overflow and
// infinities to +-448, NaN -> 0x7f|sign, sign kept on values rounding to
// zero (the code set of evo.cpp `src/fp8.cpp:26-58`), computed from the
// binade: subnormals as rint(m * 2^9), normals as rint(m * 2^(3-e)) offset
// by the exponent field.
__host__ __device__ inline uint8_t encode_e4m3(const float value) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, value);
  const uint8_t sign = (bits >> 24U) & 0x80U;
  const uint32_t abs_bits = bits & 0x7fffffffU;
  if (abs_bits > 0x7f800000U)
    return sign | 0x7fU;
  const float magnitude = __builtin_bit_cast(float, abs_bits);
  if (magnitude >= 448.0F)
    return sign | 0x7eU;
  if (magnitude < 0.015625F) {  // below 2^-6: subnormal step 2^-9
    return sign | static_cast<uint8_t>(rintf(magnitude * 512.0F));
  }
  const int exponent = static_cast<int>(abs_bits >> 23U) - 127;  // -6..8
  const float scaled = ldexpf(magnitude, 3 - exponent);          // [8, 16)
  const int q = static_cast<int>(rintf(scaled));                 // 8..16
  return sign | static_cast<uint8_t>(((exponent + 7) << 3) + (q - 8));
}

// ---- Activation storage type of the inter-kernel tensors.
enum class IoType : int { kF32 = 0, kBF16 = 1 };

// Raw buffer loads: a wave-uniform resource (base, byte bound) plus a 32-bit
// per-lane byte offset and a wave-uniform scalar byte offset, one
// buffer_load per element with no per-lane address arithmetic. Offsets at
// or past the bound read 0.
__device__ inline __amdgpu_buffer_rsrc_t buffer_resource(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}

template <typename T>
__device__ inline float buffer_act(__amdgpu_buffer_rsrc_t resource, uint32_t lane_offset,
                                   uint32_t uniform_offset) {
  if constexpr (sizeof(T) == 2)
    return bf16_to_f32(static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(
        resource, static_cast<int>(lane_offset), static_cast<int>(uniform_offset), 0)));
  else
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
        resource, static_cast<int>(lane_offset), static_cast<int>(uniform_offset), 0));
}

template <typename T> __device__ inline float load_act(const T *p, size_t i);
template <> __device__ inline float load_act<float>(const float *p, size_t i) {
  return p[i];
}
template <>
__device__ inline float load_act<uint16_t>(const uint16_t *p, size_t i) {
  return bf16_to_f32(p[i]);
}
// Stores of producer kernels (SplitOut is declared in ops.hpp).
__device__ inline void put(float *out, size_t i, float v) { out[i] = v; }
__device__ inline void put(uint16_t *out, size_t i, float v) { out[i] = f32_to_bf16(v); }
__device__ inline void put(const SplitOut &out, size_t i, float v) {
  const uint16_t hi = f32_to_bf16(v);
  out.hi[i] = hi;
  if (out.lo != nullptr)
    out.lo[i] = f32_to_bf16(v - bf16_to_f32(hi));
}

__device__ inline uint16_t f32_to_f16_sat(const float v) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(fminf(fmaxf(v, -65504.0F), 65504.0F)));
}
// Raises kFlagF16Range in *flag (when given) for a value outside the FP16
// range or NaN, which the saturating conversion would hide.
__device__ inline void note_f16_range(int *flag, float v) {
  if (flag != nullptr && !(__builtin_fabsf(v) <= 65504.0F))
    atomicOr(flag, kFlagF16Range);
}
__device__ inline void put(const F16Out &out, size_t i, float v) {
  note_f16_range(out.saturated, v);
  out.out[i] = f32_to_f16_sat(v);
}

// Non-temporal variants for outputs no later part of the producing kernel
// reads: the stores stream past the L2 instead of evicting its input lines.
__device__ inline void put_nt(float *out, size_t i, float v) {
  __builtin_nontemporal_store(v, out + i);
}
__device__ inline void put_nt(uint16_t *out, size_t i, float v) {
  __builtin_nontemporal_store(f32_to_bf16(v), out + i);
}
__device__ inline void put_nt(const F16Out &out, size_t i, float v) {
  note_f16_range(out.saturated, v);
  __builtin_nontemporal_store(f32_to_f16_sat(v), out.out + i);
}
__device__ inline void put_nt(const SplitOut &out, size_t i, float v) {
  const uint16_t hi = f32_to_bf16(v);
  __builtin_nontemporal_store(hi, out.hi + i);
  if (out.lo != nullptr)
    __builtin_nontemporal_store(f32_to_bf16(v - bf16_to_f32(hi)), out.lo + i);
}

inline Status hip_status(const hipError_t error, const char *what) {
  if (error == hipSuccess)
    return Status::Ok();
  return {ErrorCode::kHip, std::string(what) + ": " + hipGetErrorString(error)};
}

inline Status launch_status(const char *kernel) {
  return hip_status(hipGetLastError(), kernel);
}

inline unsigned ceil_div(const size_t a, const size_t b) {
  return static_cast<unsigned>((a + b - 1) / b);
}

}  // namespace evo::hip
