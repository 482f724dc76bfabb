// Shared host/device plumbing for the HiF8 HIP kernels: error reporting for the
// C ABI, dtype helpers, conversions and wavefront reductions for gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hif8_format.h"
#include "hif8_rocm.h"

namespace hif8 {

// ---------------------------------------------------------------- host side

// Records a printf-style message as this thread's last error and returns code.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Converts a pending launch error into a status; "what" names the operator.
int check_launch(const char *what);
// Clears this thread's last error (called on entry of every ABI function).
void clear_error();
// Raises the dynamic-LDS limit of `kernel` on the current device to at least
// `bytes` (hipFuncSetAttribute once per kernel, device and larger size;
// serialised by a mutex, so concurrent first launches from several host
// threads are safe).  Returns HIF8_OK or a launch error naming `what`.
int reserve_dynamic_lds(const void *kernel, size_t bytes, const char *what);

inline bool is_io_dtype(int d) { return d == HIF8_DTYPE_FP16 || d == HIF8_DTYPE_BF16; }
inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// The constexpr-built tables in device global memory (one ~9.5 KiB copy per
// translation unit; kernels stage the part they need into LDS).
static __device__ const Tables kDeviceTables = make_tables();

// ---------------------------------------------------------------- device side

constexpr int kWave = 64;

template <bool kBf16>
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  if constexpr (kBf16) {
    return __uint_as_float(h << 16);
  } else {
    return float(__builtin_bit_cast(_Float16, uint16_t(h)));
  }
}

// Low / high 16-bit lane of a packed pair to float.
template <bool kBf16>
__device__ __forceinline__ float lo_to_float(uint32_t w) {
  if constexpr (kBf16) return __uint_as_float(w << 16);
  return float(__builtin_bit_cast(_Float16, uint16_t(w & 0xFFFFu)));
}
template <bool kBf16>
__device__ __forceinline__ float hi_to_float(uint32_t w) {
  if constexpr (kBf16) return __uint_as_float(w & 0xFFFF0000u);
  return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16)));
}

// Round-to-nearest-even conversions (gfx950 v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint16_t float_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
template <bool kBf16>
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  if constexpr (kBf16) return float_to_bf16_bits(f);
  return float_to_f16_bits(f);
}

// Workgroup barrier that waits for this wave's LDS traffic only (lgkmcnt(0);
// vmcnt and expcnt left at their maxima), so global loads issued before it
// stay in flight across the barrier.  Only LDS data is exchanged through it.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no compiler motion of memory ops across
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

typedef __attribute__((address_space(3))) void lds_void_t;

// 32-bit LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return uint32_t(uintptr_t((const lds_void_t *)p));
}

// Asynchronous copy of 16 bytes per lane from global memory into LDS
// (global_load_lds_dwordx4): lane i's bytes land at lds_base + 16 * i, the
// LDS address being taken from M0 when the instruction issues.  Written as
// inline assembly so that the compiler neither waits on it nor counts it:
// every consumer of the copied data waits for it explicitly (wait_vmcnt).
// M0 is saved and restored around the copy; one wait state separates the M0
// write from the load.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds_base) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_base);  // wave-uniform: an SGPR
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(base)
      : "memory");
}

// dma16 with a wave-uniform 64-bit base (SGPRs) and a 32-bit per-lane byte
// offset: lane i's 16 bytes come from base + voffset.
__device__ __forceinline__ void dma16_offset(const void *base, uint32_t voffset, uint32_t lds_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_base);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voffset), "s"(base), "s"(lds)
      : "memory");
}

// s_waitcnt with vmcnt(n) only (lgkmcnt / expcnt left at their maxima).
template <int kN>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(kN >= 0 && kN < 64, "vmcnt range");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((kN & 0xF) | (0x7 << 4) | (0xF << 8) | ((kN >> 4) << 14));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) v += __shfl_xor(v, offset, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, kWave));
  return v;
}

}  // namespace hif8
