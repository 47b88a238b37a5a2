// Shared host/device helpers for the gfx950 kernels of libksdraft_amd.so.
//
// Numerics conventions used by every kernel (they make the int8 codes, fp16 scales
// and fp16 intermediates bit-identical to the reference's torch CPU semantics):
//   - the library is compiled with -ffp-contract=off, so a*b+c is two roundings
//     unless written as fmaf();
//   - fp32 division is IEEE correctly rounded (-fhip-fp32-correctly-rounded-divide-sqrt);
//   - fp32 -> fp16 uses _Float16 conversion (round-to-nearest-even, subnormals kept);
//   - rintf() is round-half-to-even, the rounding of torch.round.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/ksdraft_amd.h"

namespace ksd {

// ---------------------------------------------------------------- errors
// One message buffer per host thread: entry points stay reentrant.
inline thread_local char g_err[512];

inline int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

inline int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KSD_EHIP, "%s: %s", what, hipGetErrorString(e));
  return KSD_OK;
}

inline bool valid_group(int g) { return g == 32 || g == 64 || g == 128; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- device numerics
constexpr float kScaleMin = 5.9604644775390625e-08f;  // 2**-24, quant.py:22
constexpr float kScaleMax = 65504.0f;                 // quant.py:23

// Materialise v as an fp32 register value. Without this the backend may fuse the op
// that produced v with the narrowing to fp16 (e.g. fma + cvt -> v_fma_mixlo_f16), which
// rounds once instead of twice (fp32, then fp16) and differs on fp16 ties.
__device__ __forceinline__ float opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ float f16_round(float v) {  // fp32 -> fp16 -> fp32
  return (float)(_Float16)opaque(v);
}
__device__ __forceinline__ uint16_t f16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)opaque(v));
}
__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// fp32 -> bf16 round-to-nearest-even (NaN kept quiet), torch's conversion.
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int DT> struct Elem;
template <> struct Elem<KSD_F32> {
  using T = float;
  __device__ __forceinline__ static float load(const T *p) { return *p; }
};
template <> struct Elem<KSD_BF16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T *p) { return bf16_to_f32(*p); }
};
template <> struct Elem<KSD_F16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T *p) { return f16_to_f32(*p); }
};

// NaN semantics follow torch's quantize_last_dim on the CPU: amax propagates NaN, the
// NaN then passes through clamp, its fp16 scale is stored as 0x7fff, and the NaN codes
// convert to 0 (tests/test_oracle_quant.py pins this against torch).

// max of two magnitudes (sign bits clear) that propagates NaN: for non-negative floats
// the IEEE order is the integer order of the bit patterns, and NaNs sort above inf.
__device__ __forceinline__ float amax2(float a, float b) {
  return __builtin_bit_cast(float, max(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)));
}

// GS scale of a group from its amax: clamp(amax/127, 2^-24, 65504) rounded through
// fp16 (quant.py:48-49; ks3_triton.py:33-35).
__device__ __forceinline__ float group_scale(float amax) {
  float s = amax / 127.0f;
  s = s != s ? s : fminf(fmaxf(s, kScaleMin), kScaleMax);
  return f16_round(s);
}

// fp16 bits of a group scale (0x7fff for NaN, torch's fp16 conversion of that NaN).
__device__ __forceinline__ uint16_t scale_bits(float s) { return s != s ? 0x7fff : f16_bits(s); }

// clamp(round_half_even(v), -127, 127) as an int code (quant.py:50); NaN -> 0.
__device__ __forceinline__ int8_t code_of(float v) {
  float r = rintf(v);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return v != v ? (int8_t)0 : (int8_t)(int)r;
}

// Store one fp32 value as the output element type.
template <int DT> __device__ __forceinline__ void store_out(void *y, int64_t idx, float v);
template <> __device__ __forceinline__ void store_out<KSD_F32>(void *y, int64_t idx, float v) {
  ((float *)y)[idx] = v;
}
template <> __device__ __forceinline__ void store_out<KSD_BF16>(void *y, int64_t idx, float v) {
  ((uint16_t *)y)[idx] = f32_to_bf16(v);
}
template <> __device__ __forceinline__ void store_out<KSD_F16>(void *y, int64_t idx, float v) {
  ((uint16_t *)y)[idx] = f16_bits(v);
}
// fp16 then clamp(+-65504): ks3_int8.py:242 `.to(FP16).clamp(-65504., 65504.)`.
template <> __device__ __forceinline__ void store_out<KSD_F16_SAT>(void *y, int64_t idx, float v) {
  _Float16 h = (_Float16)opaque(v);
  float hf = (float)h;
  if (hf > kScaleMax) h = (_Float16)kScaleMax;
  if (hf < -kScaleMax) h = (_Float16)(-kScaleMax);
  ((uint16_t *)y)[idx] = __builtin_bit_cast(uint16_t, h);
}

}  // namespace ksd
