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

// The device's CU count (persistent launches size their grids by it), cached per device.
static inline int cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
  }
  return n;
}

// ks3.hip: launches the fused contract's per-chart increment table kernel (F x 256 fp32).
int ks3_fused_table(const int8_t *spine_codes, const uint16_t *spine_scale, const uint16_t *warp_scale,
                    const uint16_t *warp_shift, const int8_t *tanh_lut, int64_t F, float *table,
                    hipStream_t st);

// ---------------------------------------------------------------- device numerics
constexpr float kScaleMin = 5.9604644775390625e-08f;  // 2**-24, quant.py:22
constexpr float kScaleMax = 65504.0f;                 // quant.py:23

// The KS3 tanh LUT's index domain (shared by the spine kernels and the fused projection GEMM).
constexpr float kLutScale = (float)(127.0 / 3.2);   // _lut_index, ks3_int8.py:71
constexpr float kLutDomain = 3.2f;                  // TANH_DOMAIN, ks3_int8.py:46
// _lut_index_f32 of the fused kernel (ks3_triton.py:56): fp32 throughout.
__device__ __forceinline__ int lut_index_f32(float v) {
  return (int)rintf(__builtin_amdgcn_fmed3f(v, -kLutDomain, kLutDomain) * kLutScale);
}

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
// fp32 -> bf16 round-to-nearest-even (NaN kept quiet), torch's conversion; branch-free.
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)(v != v ? (u >> 16) | 0x40u : r);
}
// fp32 -> bf16 -> fp32 (round-to-nearest-even; a NaN stays a NaN).
__device__ __forceinline__ float bf16_round(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const float r = __builtin_bit_cast(float, (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
  return v != v ? v : r;
}

// Two fp32 values through bf16 and back with one v_cvt_pk_bf16_f32 (round-to-nearest-even,
// denormals kept under the kernels' fp32 denormal mode; a NaN stays a NaN).
__device__ __forceinline__ void bf16_round2(float &a, float &b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const f32x2 r = __builtin_convertvector(__builtin_convertvector((f32x2){a, b}, bf16x2), f32x2);
  a = r.x;
  b = r.y;
}

// NaN-propagating max of |v[0..n)| as fp32 (v_maximum3_f32 with abs modifiers); the result
// has its sign bit clear, so its u32 pattern orders like the magnitude, NaN above inf.
template <int N>
__device__ __forceinline__ float abs_max(const float *v) {
  float m = fabsf(v[0]);
#pragma unroll
  for (int i = 1; i + 1 < N; i += 2)
    m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(fabsf(v[i]), fabsf(v[i + 1])));
  if constexpr (N % 2 == 0) m = __builtin_elementwise_maximum(m, fabsf(v[N - 1]));
  return fabsf(m);
}

// Max of the u32 patterns over aligned groups of L lanes (L = 1, 2, 4, 8 or 16), every
// lane of a group getting the result: DPP quad permutes for the pairs and quads, then
// the half-row and row mirrors, which pair each quad (each half-row) with the other one.
template <int L>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  static_assert(L == 1 || L == 2 || L == 4 || L == 8 || L == 16, "group of 1..16 lanes");
  if constexpr (L >= 2) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  if constexpr (L >= 4) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  if constexpr (L >= 8) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  if constexpr (L >= 16) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
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

// x / 127, correctly rounded, without the division sequence: q0 = x * RN(1/127) and one
// FMA correction step with the exact residual x - 127 * q0. Checked against the IEEE
// quotient over every positive normal fp32 x (and, in tests/test_oracle_div127.py, whole
// binades of both signs, zeros, subnormals, infinities and NaNs); an infinite x, whose
// residual is NaN, keeps q0 = +-inf.
__device__ __forceinline__ float div127(float x) {
  constexpr float r = 1.0f / 127.0f;
  const float q0 = x * r;
  const float q1 = fmaf(fmaf(-q0, 127.0f, x), r, q0);
  return __builtin_isfinite(q1) ? q1 : q0;
}

// GS scale of a group from its amax: clamp(amax/127, 2^-24, 65504) rounded through
// fp16 (quant.py:48-49; ks3_triton.py:33-35).
__device__ __forceinline__ float group_scale(float amax) {
  float s = div127(amax);
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

// Distance from v to the nearest half-integer, |fract(v) - 0.5| (v_fract_f32: v - floor(v),
// exact for finite v; exact subtraction wherever the result is below 0.25). Equal to
// ||v - rint(v)| - 0.5|; a NaN v gives NaN, which fminf then ignores.
__device__ __forceinline__ float half_dist(float v) {
  return fabsf(__builtin_amdgcn_fractf(v) - 0.5f);
}

// code_of(x[j] / s) for NV values of one group, s being that group's scale from the
// NaN-propagating amax over values that include these x (so s is NaN exactly when one of
// them is, and then every code is 0, as x / NaN is). Otherwise s lies in [2^-24, 65504]
// and a reciprocal multiply replaces the correctly rounded division: r = rcp(s) is within
// 1 ulp of 1/s, so p = x * r is within 1.5 * 2^-23 relative of the real quotient, which is
// below 1.5 * 2^-16 absolute wherever |p| <= 128 (beyond that both sides clamp to +-127).
// rint(p) therefore equals rint(x / s) unless p lies within 2^-15 of a half-integer
// (half-integers below 2^22 are fp32 values, so the rounded division cannot cross one
// either). A lane with any p within 2^-14 of a half-integer recomputes its NV codes with
// the division.
template <int NV>
__device__ __forceinline__ void codes_rcp(const float *x, float s, int8_t *q) {
  if (s != s) {
#pragma unroll
    for (int j = 0; j < NV; ++j) q[j] = 0;
    return;
  }
  const float r = __builtin_amdgcn_rcpf(s);
  bool near_tie = false;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float p = x[j] * r;
    const float t = rintf(p);
    near_tie |= fabsf(fabsf(p - t) - 0.5f) < 0x1p-14f;
    q[j] = (int8_t)(int)fminf(fmaxf(t, -127.0f), 127.0f);   // t is integral or +-inf
  }
  if (near_tie) {
#pragma unroll
    for (int j = 0; j < NV; ++j) q[j] = code_of(x[j] / s);
  }
}

// code_of(x[j] / s) for NV values of one group (NV a multiple of 4), packed four to a word,
// little-endian. s is that group's scale from the NaN-propagating amax over values that
// include these x: it is NaN exactly when one of them is, and then every code is 0 (as
// x / NaN is). Otherwise s lies in [2^-24, 65504] and a reciprocal multiply replaces the
// correctly rounded division. r = rcp(s) is within 1 ulp of 1/s, so p = x * r is within
// 1.5 * 2^-23 relative of the real quotient: below 1.5 * 2^-16 absolute wherever |p| <= 128
// (beyond that both sides clamp to +-127), and the rounded quotient is within 2^-18 of the
// real one. rint(p) therefore equals rint(x / s) unless p lies within 2^-15 of a
// half-integer; an 8-code chunk holding any p within 2^-14 of one is recomputed with the
// division (the branch is rarely taken by a whole wave, so it stays cheap on average).
// Rounding and clamping go through one add: for |c| <= 127, c + 1.5 * 2^23 rounds c to the
// nearest integer (ties to even) and leaves it, two's complement, in the low byte of the
// sum's bit pattern; v_perm_b32 then gathers four low bytes. Clamping before the rounding
// equals clamping after it, +-127 being integers.
template <int NV>
__device__ __forceinline__ void codes_rcp_packed(const float *x, float s, uint32_t *w) {
  static_assert(NV % 4 == 0, "whole words");
  if (s != s) {
#pragma unroll
    for (int k = 0; k < NV / 4; ++k) w[k] = 0;
    return;
  }
  constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
  constexpr int CH = NV < 8 ? NV : 8;
  const float r = __builtin_amdgcn_rcpf(s);
  uint32_t f[NV];
#pragma unroll
  for (int c0 = 0; c0 < NV; c0 += CH) {
    float near = 1.0f;
#pragma unroll
    for (int j = c0; j < c0 + CH; ++j) {
      const float c = __builtin_amdgcn_fmed3f(x[j] * r, -127.0f, 127.0f);
      const float m = c + kMagic;
      near = fminf(near, half_dist(c));
      f[j] = __builtin_bit_cast(uint32_t, m);
    }
    if (near < 0x1p-14f) {
#pragma unroll
      for (int j = c0; j < c0 + CH; ++j) f[j] = (uint8_t)code_of(x[j] / s);
    }
  }
#pragma unroll
  for (int k = 0; k < NV / 4; ++k)
    w[k] = __builtin_amdgcn_perm(f[4 * k + 1], f[4 * k], 0x0c0c0400u) |
           __builtin_amdgcn_perm(f[4 * k + 3], f[4 * k + 2], 0x04000c0cu);
}

// Raw buffer resources: a lane whose offset lies at or past num_records reads zeros and
// its stores are dropped, which masks ragged rows and columns without branches.
constexpr int kBufFlags = 0x00020000;
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0,
                                           (int)min(bytes, (int64_t)0x7fffffff), kBufFlags);
}

// 8 consecutive elements as raw bits: two 16-byte vectors for fp32, one for 16-bit types.
template <int DT> struct Raw8 { uint4 a, b; };
template <int DT>
__device__ __forceinline__ Raw8<DT> load_raw8(const typename Elem<DT>::T *p) {
  Raw8<DT> r;
  r.a = *(const uint4 *)p;
  if constexpr (DT == KSD_F32) r.b = *(const uint4 *)(p + 4);
  return r;
}
template <int DT>
__device__ __forceinline__ void cvt_raw8(const Raw8<DT> &r, bool ok, float *v) {
  const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float f;
    if constexpr (DT == KSD_F32) {
      f = __builtin_bit_cast(float, w[i]);
    } else {
      const uint16_t h = (uint16_t)(i & 1 ? w[i / 2] >> 16 : w[i / 2] & 0xffffu);
      f = Elem<DT>::load(&h);
    }
    v[i] = ok ? f : 0.0f;
  }
}

// An fp32 value rounded to the element type DT and back (identity for fp32).
template <int DT>
__device__ __forceinline__ float round_to_dt(float v);
template <> __device__ __forceinline__ float round_to_dt<KSD_F32>(float v) { return v; }
template <> __device__ __forceinline__ float round_to_dt<KSD_BF16>(float v) { return bf16_round(v); }
template <> __device__ __forceinline__ float round_to_dt<KSD_F16>(float v) { return f16_round(v); }

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
