// KS3 int8 cell kernels for gfx950: the composed (training) contract of
// ksdraft/kernels/ks3_int8.py, rank 1.
//
//   ks3_spine_kernel   _spine_features 'int8' mode (ks3_int8.py:205-234) on the fp16
//                      coordinates of _project (:241-242), fused with the per-group
//                      quantize_last_dim(h, group) that follows it (:330 / :309).
//   ks3_vjp_kernel     the fp16 geometry VJP of _KS3Int8Train.backward (:354-401): dc in
//                      fp16 and directly as the two int8 operands the backward GEMMs need
//                      (quantized along F for dx, :410; along M for ddown, :417), plus
//                      per-block column partial sums of the eight reductions (:379-388).
//   ks3_vjp_finalize   fixed-order sum of those partials, fp16 rounding, STE chain (:389-395).
//
// fp16 semantics: every fp16 tensor op of the reference is an fp32 evaluation rounded to
// fp16. For + - * on fp16 operands that equals the native fp16 instruction (fp32 keeps
// 24 >= 2*11+2 bits, so rounding twice equals rounding once), so the VJP runs on packed
// fp16 (v_pk_*_f16), two rows of one column per register. tanh takes an fp16 argument and
// is read from a table of round_fp16(round_fp32(tanh(x))) over all fp16 inputs, the
// function torch computes on fp16 tensors.
#include "ksd_common.h"
#include "tanh16_table.inc"

namespace ksd {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr float kLutScale = (float)(127.0 / 3.2);   // _lut_index, ks3_int8.py:71
constexpr float kLutDomain = 3.2f;                  // TANH_DOMAIN, ks3_int8.py:46
constexpr float kTq16Step = (float)(4.0 / 127.0);   // ks3_int8.py:211

// ---------------------------------------------------------------- integer helpers
// _round_div127 (ks3_int8.py:57-66): truncating quotient, +-1 when |remainder| > 63.
__device__ __forceinline__ int round_div127(int v) {
  int q = v / 127;
  int r = v - q * 127;
  return q + (r > 63 ? 1 : (r < -63 ? -1 : 0));
}

// _lut_index (ks3_int8.py:69-72) of an fp16 value: clamp (fp16 result), * 127/3.2
// rounded to fp16, round half to even.
__device__ __forceinline__ int lut_index(float x16) {
  float c = f16_round(fminf(fmaxf(x16, -kLutDomain), kLutDomain));
  return (int)rintf(f16_round(c * kLutScale));
}

__device__ __forceinline__ int lut_at(const int8_t *lut, int i) {
  i += 128;
  i = i < 0 ? 0 : (i > 255 ? 255 : i);
  return lut[i];
}


// ---------------------------------------------------------------- spine forward
// Column constants of the integer Horner (ks3_int8.py:214-225), pre-multiplied by 64.
struct SpineCol {
  int a64, b64, c2_64, c0_64, c5x4_64, c4x2_64, c5x3_64, c4_64;
  float ps, sc, sh;
};

__device__ __forceinline__ SpineCol load_spine_col(const int8_t *codes, const uint16_t *ps,
                                                   const uint16_t *sc16, const uint16_t *sh16,
                                                   int64_t f, bool valid) {
  SpineCol c;
  if (!valid) {
    c.a64 = c.b64 = c.c2_64 = c.c0_64 = c.c5x4_64 = c.c4x2_64 = c.c5x3_64 = c.c4_64 = 0;
    c.ps = c.sc = c.sh = 0.0f;
    return c;
  }
  const int8_t *p = codes + f * 6;
  int c0 = p[0], c1 = p[1], c2 = p[2], c3 = p[3], c4 = p[4], c5 = p[5];
  c.a64 = (2 * c0 - 2 * c1 + c2 + c3) * 64;
  c.b64 = (-3 * c0 + 3 * c1 - 2 * c2 - c3) * 64;
  c.c2_64 = c2 * 64;
  c.c0_64 = c0 * 64;
  c.c5x4_64 = 4 * c5 * 64;
  c.c4x2_64 = 2 * c4 * 64;
  c.c5x3_64 = 3 * c5 * 64;
  c.c4_64 = c4 * 64;
  c.ps = f16_to_f32(ps[f]);
  c.sc = f16_to_f32(sc16[f]);
  c.sh = f16_to_f32(sh16[f]);
  return c;
}

// One feature of _spine_features 'int8' mode, rank 1 (mean == x). Returns the fp32
// ReLU^2 feature fp16(hq*hq) * pre^2.
__device__ __forceinline__ float spine_feature(float x, const SpineCol &c, const int8_t *lut) {
  int ti = lut_index(f16_round(x * 0.25f));
  int tq = lut_at(lut, ti);
  float w = f16_round(f16_round((float)tq * kTq16Step) + c.sh);
  w = f16_round(c.sc * w);
  int zq = lut_at(lut, lut_index(w));
  int poly = c.a64;
  poly = round_div127(poly * tq * 4) + c.b64;
  poly = round_div127(poly * tq * 4) + c.c2_64;
  poly = round_div127(poly * tq * 4) + c.c0_64;
  int wp = c.c5x4_64;
  wp = round_div127(wp * zq) + c.c4x2_64;
  wp = round_div127(wp * zq) - c.c5x3_64;
  wp = round_div127(wp * zq) - c.c4_64;
  int td = (poly + wp) / 64;  // torch.div(..., rounding_mode="trunc")
  float h = x + f16_round(f16_round((float)td) * c.ps);
  h = h < 0.0f ? 0.0f : h;  // relu
  float pre = group_scale(fabsf(h));  // amax over the rank dim (one element), ks3_int8.py:230-231
  float q = fminf(fmaxf(rintf(h / pre), -127.0f), 127.0f);
  q = fmaxf(q, 0.0f);
  return f16_round(q * q) * (pre * pre);
}

// Block: 256 threads = 8 rows x 32 lanes; a lane owns 4 consecutive columns of a
// 128-column segment (blockIdx.x). Rows [blockIdx.y * kSpineRows, +kSpineRows).
constexpr int kSpineRows = 64;

template <int G, bool VEC>
__global__ void __launch_bounds__(256) ks3_spine_kernel(
    const uint16_t *__restrict__ coords, int64_t M, int64_t F,
    const int8_t *__restrict__ spine_codes, const uint16_t *__restrict__ spine_scale,
    const uint16_t *__restrict__ sc16, const uint16_t *__restrict__ sh16,
    const int8_t *__restrict__ tanh_lut, float *__restrict__ h_out,
    int8_t *__restrict__ hq, uint16_t *__restrict__ hs, int64_t n_groups) {
  __shared__ int8_t lut[256];
  if (threadIdx.x < 64) ((uint32_t *)lut)[threadIdx.x] = ((const uint32_t *)tanh_lut)[threadIdx.x];
  const int lane = threadIdx.x & 31;
  const int rsub = threadIdx.x >> 5;
  const int64_t col0 = (int64_t)blockIdx.x * 128 + lane * 4;
  SpineCol cc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    cc[j] = load_spine_col(spine_codes, spine_scale, sc16, sh16, col0 + j, col0 + j < F);
  __syncthreads();

  const int64_t row_end = min(M, (int64_t)(blockIdx.y + 1) * kSpineRows);
  for (int64_t row = (int64_t)blockIdx.y * kSpineRows + rsub; row < row_end; row += 8) {
    float x[4];
    const uint16_t *src = coords + row * F + col0;
    if (VEC && col0 + 3 < F) {
      uint2 u = *(const uint2 *)src;
      x[0] = f16_to_f32((uint16_t)u.x);
      x[1] = f16_to_f32((uint16_t)(u.x >> 16));
      x[2] = f16_to_f32((uint16_t)u.y);
      x[3] = f16_to_f32((uint16_t)(u.y >> 16));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = col0 + j < F ? f16_to_f32(src[j]) : 0.0f;
    }
    float h[4];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h[j] = col0 + j < F ? spine_feature(x[j], cc[j], lut) : 0.0f;
      amax = amax2(amax, fabsf(h[j]));
    }
    if (h_out) {
      float *dst = h_out + row * F + col0;
      if (VEC && col0 + 3 < F) {
        *(float4 *)dst = make_float4(h[0], h[1], h[2], h[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (col0 + j < F) dst[j] = h[j];
      }
    }
    if (hq) {
      // quantize_last_dim(h, G): one group = G/4 lanes
#pragma unroll
      for (int o = 1; o < G / 4; o <<= 1) amax = amax2(amax, __shfl_xor(amax, o, 32));
      const float s = group_scale(amax);
      int8_t q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) q[j] = code_of(h[j] / s);
      int8_t *dst = hq + row * F + col0;
      if (VEC && col0 + 3 < F) {
        *(uint32_t *)dst = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
                           ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (col0 + j < F) dst[j] = q[j];
      }
      if ((lane & (G / 4 - 1)) == 0 && col0 < F) hs[row * n_groups + col0 / G] = scale_bits(s);
    }
  }
}


// The fused-kernel contract of project_fused / _fused_gemm_spine, 'int8' mode
// (ks3_triton.py:47-75, 137-156). It differs from the composed one: x is the fp32 GEMM
// accumulator clamped to +-65504 (no fp16 materialisation); LUT indices are computed in
// fp32; the Horner sum is scaled by ps/64 in fp32 without truncation; the ReLU^2 pre-scale
// is the amax of |h| (before ReLU) over the row's G-chart group; the squared codes are
// exact; and the result is requantized per group a second time.
__device__ __forceinline__ int lut_index_f32(float v) {
  return (int)rintf(fminf(fmaxf(v, -kLutDomain), kLutDomain) * kLutScale);
}

__device__ __forceinline__ float spine_fused_h(float x, const SpineCol &c, const int8_t *lut) {
  int tq = lut_at(lut, lut_index_f32(x * 0.25f));
  float w = f16_round(f16_round((float)tq * kTq16Step) + c.sh);
  w = f16_round(c.sc * w);
  int zq = lut_at(lut, lut_index_f32(w));
  int poly = c.a64;
  poly = round_div127(poly * tq * 4) + c.b64;
  poly = round_div127(poly * tq * 4) + c.c2_64;
  poly = round_div127(poly * tq * 4) + c.c0_64;
  int wp = c.c5x4_64;
  wp = round_div127(wp * zq) + c.c4x2_64;
  wp = round_div127(wp * zq) - c.c5x3_64;
  wp = round_div127(wp * zq) - c.c4_64;
  return x + (float)(poly + wp) * (c.ps / 64.0f);
}

template <int G, bool VEC>
__global__ void __launch_bounds__(256) ks3_spine_fused_kernel(
    const float *__restrict__ acc, int64_t M, int64_t F,
    const int8_t *__restrict__ spine_codes, const uint16_t *__restrict__ spine_scale,
    const uint16_t *__restrict__ sc16, const uint16_t *__restrict__ sh16,
    const int8_t *__restrict__ tanh_lut, int8_t *__restrict__ hq, uint16_t *__restrict__ hs,
    int64_t n_groups) {
  __shared__ int8_t lut[256];
  if (threadIdx.x < 64) ((uint32_t *)lut)[threadIdx.x] = ((const uint32_t *)tanh_lut)[threadIdx.x];
  const int lane = threadIdx.x & 31;
  const int rsub = threadIdx.x >> 5;
  const int64_t col0 = (int64_t)blockIdx.x * 128 + lane * 4;
  SpineCol cc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    cc[j] = load_spine_col(spine_codes, spine_scale, sc16, sh16, col0 + j, col0 + j < F);
  __syncthreads();

  const int64_t row_end = min(M, (int64_t)(blockIdx.y + 1) * kSpineRows);
  for (int64_t row = (int64_t)blockIdx.y * kSpineRows + rsub; row < row_end; row += 8) {
    float x[4];
    const float *src = acc + row * F + col0;
    if (VEC && col0 + 3 < F) {
      float4 u = *(const float4 *)src;
      x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = col0 + j < F ? src[j] : 0.0f;
    }
    float h[4];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float xc = fminf(fmaxf(x[j], -kScaleMax), kScaleMax);
      h[j] = col0 + j < F ? spine_fused_h(xc, cc[j], lut) : 0.0f;
      amax = amax2(amax, fabsf(h[j]));
    }
#pragma unroll
    for (int o = 1; o < G / 4; o <<= 1) amax = amax2(amax, __shfl_xor(amax, o, 32));
    const float pre = group_scale(amax);
    float hmax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float q = fmaxf(fminf(fmaxf(rintf(h[j] / pre), -127.0f), 127.0f), 0.0f);
      h[j] = (q * q) * (pre * pre);
      hmax = amax2(hmax, fabsf(h[j]));
    }
#pragma unroll
    for (int o = 1; o < G / 4; o <<= 1) hmax = amax2(hmax, __shfl_xor(hmax, o, 32));
    const float s = group_scale(hmax);
    int8_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = code_of(h[j] / s);
    int8_t *dst = hq + row * F + col0;
    if (VEC && col0 + 3 < F) {
      *(uint32_t *)dst = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
                         ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (col0 + j < F) dst[j] = q[j];
    }
    if ((lane & (G / 4 - 1)) == 0 && col0 < F) hs[row * n_groups + col0 / G] = scale_bits(s);
  }
}

// ---------------------------------------------------------------- VJP
// fp16 tanh of two packed fp16 values through the LDS table.
__device__ __forceinline__ h2 tanh2(h2 a, const uint16_t *tab) {
  uint32_t u = __builtin_bit_cast(uint32_t, a);
  uint32_t m0 = min(u & 0x7fffu, (uint32_t)KSD_TANH16_LIMIT);
  uint32_t m1 = min((u >> 16) & 0x7fffu, (uint32_t)KSD_TANH16_LIMIT);
  uint32_t r = (uint32_t)tab[m0] | ((uint32_t)tab[m1] << 16);
  return __builtin_bit_cast(h2, r | (u & 0x80008000u));
}

__device__ __forceinline__ h2 bc(_Float16 v) { return (h2){v, v}; }
__device__ __forceinline__ _Float16 hh(float v) { return (_Float16)opaque(v); }

// Column constants of the VJP in fp16, each the reference's fp16 tensor expression
// (ks3_int8.py:355-372) rounded op by op; a lane's two columns share one register.
struct VjpCols {
  h2 c0, c2, c4, sc, sh;
  h2 cubic, quad, c5x4, c4x2, c5x3, cubic3, quad2, c5x12, c4x4;
};

__device__ __forceinline__ void load_vjp_col(VjpCols &c, int e, const int8_t *codes, const uint16_t *ps,
                                             const uint16_t *sc16, const uint16_t *sh16,
                                             int64_t f, bool valid) {
  float k[6];
  float scale = valid ? f16_to_f32(ps[f]) : 0.0f;
#pragma unroll
  for (int i = 0; i < 6; ++i) k[i] = valid ? f16_round((float)codes[f * 6 + i] * scale) : 0.0f;
  const float c0 = k[0], c1 = k[1], c2 = k[2], c3 = k[3], c4 = k[4], c5 = k[5];
  float cubic = f16_round(f16_round(f16_round(f16_round(2.0f * c0) - f16_round(2.0f * c1)) + c2) + c3);
  float quad = f16_round(f16_round(f16_round(f16_round(-3.0f * c0) + f16_round(3.0f * c1)) -
                                   f16_round(2.0f * c2)) - c3);
  c.c0[e] = hh(c0);
  c.c2[e] = hh(c2);
  c.c4[e] = hh(c4);
  c.sc[e] = hh(valid ? f16_to_f32(sc16[f]) : 0.0f);
  c.sh[e] = hh(valid ? f16_to_f32(sh16[f]) : 0.0f);
  c.cubic[e] = hh(cubic);
  c.quad[e] = hh(quad);
  c.c5x4[e] = hh(4.0f * c5);
  c.c4x2[e] = hh(2.0f * c4);
  c.c5x3[e] = hh(3.0f * c5);
  c.cubic3[e] = hh(3.0f * cubic);
  c.quad2[e] = hh(2.0f * quad);
  c.c5x12[e] = hh(12.0f * c5);
  c.c4x4[e] = hh(4.0f * c4);
}

constexpr int kVjpTile = 128;         // rows and columns of one tile

// acc + float(t.lo) / float(t.hi), one rounding (v_fma_mix_f32 with b = 1.0).
__device__ __forceinline__ float add_lo(float acc, h2 t) {
  asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(t));
  return acc;
}
__device__ __forceinline__ float add_hi(float acc, h2 t) {
  asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(t));
  return acc;
}

// Geometry VJP of one row at two columns (packed). Accumulates the eight column terms
// into acc[k][0..1] (fp32) and returns dc = value + dmean (fp16).
__device__ __forceinline__ h2 vjp_pair(h2 v, h2 x, const VjpCols &c, const uint16_t *tab,
                                       float (*acc)[2]) {
  const h2 one = bc((_Float16)1.0f);
  const h2 t = bc((_Float16)4.0f) * tanh2(x * bc((_Float16)0.25f), tab);
  const h2 tps = t + c.sh;
  const h2 z = tanh2(c.sc * tps, tab);
  h2 spine = c.cubic * t + c.quad;
  spine = spine * t + c.c2;
  spine = spine * t + c.c0;
  h2 warped = c.c5x4 * z + c.c4x2;
  warped = warped * z - c.c5x3;
  warped = warped * z - c.c4;
  h2 pre = x + spine;
  pre = pre + warped;
  pre = pre < bc((_Float16)0.0f) ? bc((_Float16)0.0f) : pre;  // torch.relu: keeps -0 and NaN
  const h2 dpre = (v * bc((_Float16)2.0f)) * pre;
  h2 dpoly = c.cubic3 * t + c.quad2;
  dpoly = dpoly * t + c.c2;
  h2 dwarp = c.c5x12 * z + c.c4x4;
  dwarp = dwarp * z - c.c5x3;
  const h2 z2 = z * z;
  const h2 dz = dwarp * (one - z2);
  const h2 t2 = t * t;
  const h2 dmean = (dpre * (dpoly + dz * c.sc)) * (one - t2 * bc((_Float16)0.0625f));
  const h2 t3 = t2 * t;
  const h2 z3 = z2 * z;
  const h2 t3x2 = bc((_Float16)2.0f) * t3;
  const h2 t2x3 = bc((_Float16)3.0f) * t2;
  const h2 dpdz = dpre * dz;
  const h2 terms[8] = {
      dpre * ((t3x2 - t2x3) + one),
      dpre * (t2x3 - t3x2),
      dpre * ((t3 - bc((_Float16)2.0f) * t2) + t),
      dpre * (t3 - t2),
      dpre * (bc((_Float16)2.0f) * z2 - one),
      dpre * (bc((_Float16)4.0f) * z3 - bc((_Float16)3.0f) * z),
      dpdz * tps,
      dpdz * c.sc,
  };
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    acc[k][0] = add_lo(acc[k][0], terms[k]);
    acc[k][1] = add_hi(acc[k][1], terms[k]);
  }
  return v + dmean;
}

__device__ __forceinline__ h2 habs2(h2 a) {
  return __builtin_bit_cast(h2, __builtin_bit_cast(uint32_t, a) & 0x7fff7fffu);
}

// Packed max of fp16 magnitudes that propagates NaN (v_pk_max_u16 on the bit patterns;
// fp16 NaNs sort above inf), like torch's amax.
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2 hmax2(h2 a, h2 b) {
  return __builtin_bit_cast(h2, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                          __builtin_bit_cast(u16x2, b)));
}

// The rows [row0, row0 + n) of a row-major tensor, clipped at M: rows past M read zeros
// and drop stores. row0 is wave-uniform, so the descriptor lives in SGPRs.
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(T *base, int64_t row0, int n, int64_t M,
                                                            int64_t row_elems) {
  const int64_t rows = max((int64_t)0, min((int64_t)n, M - row0));
  return rsrc(base + row0 * row_elems, rows * row_elems * (int64_t)sizeof(T));
}

// Block: 256 threads (4 waves) on the 128 x 128 tile (column tile blockIdx.x, row tile
// blockIdx.y). Lane l owns columns 2l and 2l+1 of the 32 rows wave*32 + i; a register
// holds one row at both columns. VEC: F is even, so a lane's two columns are both valid
// or both past F.
template <int G, bool VEC>
__global__ void __launch_bounds__(256) ks3_vjp_kernel(
    const uint16_t *__restrict__ value, const uint16_t *__restrict__ coords, int64_t M, int64_t F,
    const int8_t *__restrict__ spine_codes, const uint16_t *__restrict__ spine_scale,
    const uint16_t *__restrict__ sc16, const uint16_t *__restrict__ sh16,
    uint16_t *__restrict__ dc_out, int8_t *__restrict__ dcq, uint16_t *__restrict__ dcs,
    int8_t *__restrict__ dctq, uint16_t *__restrict__ dcts, float *__restrict__ partials) {
  __shared__ uint16_t tab[KSD_TANH16_LIMIT + 2];
  __shared__ uint32_t colmax[4][kVjpTile / 2];  // packed fp16 column maxima per wave
  for (int i = threadIdx.x; i < (KSD_TANH16_LIMIT + 2) / 2; i += 256)
    ((uint32_t *)tab)[i] = i * 2 + 1 <= KSD_TANH16_LIMIT
                               ? (uint32_t)kTanh16[2 * i] | ((uint32_t)kTanh16[2 * i + 1] << 16)
                               : (uint32_t)kTanh16[2 * i];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t col0 = (int64_t)blockIdx.x * kVjpTile + lane * 2;
  const bool ok0 = col0 < F, ok1 = col0 + 1 < F;
  const int64_t ngF = (F + G - 1) / G, ngM = (M + G - 1) / G;
  // per-lane column offsets within a row (bytes): fp16 and int8 elements
  const uint32_t voff2 = ok0 ? (uint32_t)(col0 * 2) : kOob, voff2b = ok1 ? (uint32_t)(col0 * 2 + 2) : kOob;
  const uint32_t voff1 = ok0 ? (uint32_t)col0 : kOob, voff1b = ok1 ? (uint32_t)(col0 + 1) : kOob;
  VjpCols cc;
  load_vjp_col(cc, 0, spine_codes, spine_scale, sc16, sh16, col0, ok0);
  load_vjp_col(cc, 1, spine_codes, spine_scale, sc16, sh16, col0 + 1, ok1);
  float acc[8][2];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k][0] = acc[k][1] = 0.0f;
  // column-block bases of the transposed outputs (offsets stay below 2^31)
  int8_t *dctq_b = dctq ? dctq + (int64_t)blockIdx.x * kVjpTile * M : nullptr;
  uint16_t *dcts_b = dcts ? dcts + (int64_t)blockIdx.x * kVjpTile * ngM : nullptr;
  const int64_t cols_here = min((int64_t)kVjpTile, F - (int64_t)blockIdx.x * kVjpTile);
  __syncthreads();

  {
    const int64_t tr0 = (int64_t)blockIdx.y * kVjpTile;  // first row of the tile
    const int r0 = wave * 32;                            // first tile row of this wave
    const int64_t grow0 = tr0 + r0;                      // global row of this wave's first row
    const auto rv = rows_rsrc(value, grow0, 32, M, F);
    const auto rx = rows_rsrc(coords, grow0, 32, M, F);
    const uint32_t rstride2 = (uint32_t)(F * 2);

    h2 dc[32];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      h2 va[16], xa[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t ro = (uint32_t)(half * 16 + i) * rstride2;
        if (VEC) {
          va[i] = __builtin_bit_cast(h2, __builtin_amdgcn_raw_buffer_load_b32(rv, voff2 + ro, 0, 0));
          xa[i] = __builtin_bit_cast(h2, __builtin_amdgcn_raw_buffer_load_b32(rx, voff2 + ro, 0, 0));
        } else {
          const uint32_t o0 = voff2 + ro, o1 = voff2b + ro;
          va[i] = (h2){__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rv, o0, 0, 0)),
                       __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rv, o1, 0, 0))};
          xa[i] = (h2){__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rx, o0, 0, 0)),
                       __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rx, o1, 0, 0))};
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        dc[half * 16 + i] = vjp_pair(va[i], xa[i], cc, tab, acc);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // dc itself (fp16, row-major)
    if (dc_out) {
      const auto rd = rows_rsrc(dc_out, grow0, 32, M, F);
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const uint32_t ro = (uint32_t)i * rstride2;
        if (VEC) {
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, dc[i]), rd, voff2 + ro, 0, 0);
        } else {
          // halves through an explicit 32-bit shift: storing the vector element dc[i][1]
          // directly compiles to a store of the low half (hipcc 7.2, gfx950)
          const uint32_t w = __builtin_bit_cast(uint32_t, dc[i]);
          __builtin_amdgcn_raw_buffer_store_b16((uint16_t)w, rd, voff2 + ro, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(w >> 16), rd, voff2b + ro, 0, 0);
        }
      }
    }

    // quantize_last_dim(dc, G): groups of G columns per row (ks3_int8.py:410); a group is
    // G/2 lanes. Two rows are reduced per packed register.
    if (dcq) {
      const bool writes_scale = (lane & (G / 2 - 1)) == 0 && ok0;
      const uint32_t soff = writes_scale ? (uint32_t)(col0 / G * 2) : kOob;
      const auto rq = rows_rsrc(dcq, grow0, 32, M, F);
      const auto rsc = rows_rsrc(dcs, grow0, 32, M, ngF);
#pragma unroll
      for (int i = 0; i < 32; i += 2) {
        const h2 a0 = habs2(dc[i]), a1 = habs2(dc[i + 1]);
        h2 m = hmax2((h2){a0[0], a1[0]}, (h2){a0[1], a1[1]});
#pragma unroll
        for (int o = 1; o < G / 2; o <<= 1) {
          uint32_t u = __shfl_xor(__builtin_bit_cast(uint32_t, m), o, 64);
          m = hmax2(m, __builtin_bit_cast(h2, u));
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const uint32_t ro = (uint32_t)((i + e) * F);
          const float s = group_scale((float)m[e]);
          const uint32_t q0 = (uint8_t)code_of((float)dc[i + e][0] / s);
          const uint32_t q1 = (uint8_t)code_of((float)dc[i + e][1] / s);
          if (VEC) {
            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(q0 | (q1 << 8)), rq, voff1 + ro, 0, 0);
          } else {
            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)q0, rq, voff1 + ro, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)q1, rq, voff1b + ro, 0, 0);
          }
          __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rsc, soff + (uint32_t)((i + e) * ngF * 2), 0, 0);
        }
      }
    }

    // quantize_last_dim(dc.t(), G): groups of G rows per column (ks3_int8.py:417)
    if (dctq) {
      h2 m = habs2(dc[0]);
#pragma unroll
      for (int i = 1; i < 32; ++i) m = hmax2(m, habs2(dc[i]));
      if (G > 32) {
        colmax[wave][lane] = __builtin_bit_cast(uint32_t, m);
        __syncthreads();
        const int w0 = wave / (G / 32) * (G / 32);  // first wave of this lane's row group
        m = __builtin_bit_cast(h2, colmax[w0][lane]);
#pragma unroll
        for (int w = 1; w < G / 32; ++w)
          m = hmax2(m, __builtin_bit_cast(h2, colmax[w0 + w][lane]));
        __syncthreads();  // colmax is rewritten by the next tile
      }
      const auto rq = rsrc(dctq_b, cols_here * M);
      const auto rsc = rsrc(dcts_b, cols_here * ngM * 2);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float s = group_scale((float)m[e]);
        const bool colok = e ? ok1 : ok0;
        const int64_t lc = lane * 2 + e;  // column within the block
        uint32_t w[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          w[q] = 0;
#pragma unroll
          for (int b = 0; b < 4; ++b)
            w[q] |= (uint32_t)(uint8_t)code_of((float)dc[q * 4 + b][e] / s) << (8 * b);
        }
        if (grow0 + 32 <= M && (M & 15) == 0) {
          const uint32_t off = colok ? (uint32_t)(lc * M + grow0) : kOob;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, make_uint4(w[0], w[1], w[2], w[3])),
                                                 rq, off, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, make_uint4(w[4], w[5], w[6], w[7])),
                                                 rq, colok ? off + 16 : kOob, 0, 0);
        } else {
          for (int r = 0; r < 32; ++r) {
            const uint32_t off = colok && grow0 + r < M ? (uint32_t)(lc * M + grow0 + r) : kOob;
            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(w[r >> 2] >> (8 * (r & 3))), rq, off, 0, 0);
          }
        }
        const bool writes_scale = r0 % G == 0 && colok && grow0 < M;
        const uint32_t soff = writes_scale ? (uint32_t)((lc * ngM + grow0 / G) * 2) : kOob;
        __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rsc, soff, 0, 0);
      }
    }
  }

  // column partial sums of this block: the 4 waves hold the same columns
  __syncthreads();  // the table region is reused below
  float *red = (float *)tab;  // [4 waves][8 terms][128 cols] = 16 KiB
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    red[(wave * 8 + k) * kVjpTile + lane * 2] = acc[k][0];
    red[(wave * 8 + k) * kVjpTile + lane * 2 + 1] = acc[k][1];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 8 * kVjpTile; i += 256) {
    const int k = i / kVjpTile, c = i % kVjpTile;
    const int64_t col = (int64_t)blockIdx.x * kVjpTile + c;
    if (col >= F) continue;
    float s = red[(0 * 8 + k) * kVjpTile + c];
    s += red[(1 * 8 + k) * kVjpTile + c];
    s += red[(2 * 8 + k) * kVjpTile + c];
    s += red[(3 * 8 + k) * kVjpTile + c];
    partials[((int64_t)blockIdx.y * 8 + k) * F + col] = s;
  }
}

// Fixed-order sum of the per-block partials, then the reference's fp16 roundings and the
// STE chain to the raw warp parameters (ks3_int8.py:379-395).
__global__ void ks3_vjp_finalize_kernel(const float *__restrict__ partials, int64_t nrb, int64_t F,
                                        const float *__restrict__ raw_scale,
                                        const float *__restrict__ raw_shift, float *__restrict__ sums,
                                        uint16_t *__restrict__ dcoeff, uint16_t *__restrict__ dscale,
                                        uint16_t *__restrict__ dshift) {
  const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= F) return;
  float s[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float a = 0.0f;
    for (int64_t b = 0; b < nrb; ++b) a += partials[(b * 8 + k) * F + f];
    s[k] = a;
    if (sums) sums[k * F + f] = a;
  }
#pragma unroll
  for (int k = 0; k < 6; ++k) dcoeff[f * 6 + k] = f16_bits(s[k]);
  const float dscale_t = f16_round(s[6]);
  const float dshift_t = f16_round(f16_round(s[7]) * 0.5f);
  const float sig = 1.0f / (1.0f + expf(-raw_scale[f]));
  const float th = tanhf(raw_shift[f]);
  dscale[f] = f16_bits(dscale_t * sig);
  dshift[f] = f16_bits(dshift_t * (1.0f - th * th));
}

// fp16 tanh through the same table (test export).
__global__ void ks3_tanh16_kernel(const uint16_t *__restrict__ x, int64_t n, uint16_t *__restrict__ y) {
  __shared__ uint16_t tab[KSD_TANH16_LIMIT + 2];
  for (int i = threadIdx.x; i <= KSD_TANH16_LIMIT; i += blockDim.x) tab[i] = kTanh16[i];
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  h2 a = {__builtin_bit_cast(_Float16, x[i]), (_Float16)0.0f};
  y[i] = __builtin_bit_cast(uint16_t, tanh2(a, tab)[0]);
}

// ---------------------------------------------------------------- launchers
template <int G>
static void launch_spine(bool vec, dim3 grid, hipStream_t st, const uint16_t *coords, int64_t M,
                         int64_t F, const int8_t *sc, const uint16_t *ss, const uint16_t *w16,
                         const uint16_t *h16, const int8_t *lut, float *h, int8_t *hq, uint16_t *hs,
                         int64_t ng) {
  if (vec)
    hipLaunchKernelGGL((ks3_spine_kernel<G, true>), grid, dim3(256), 0, st, coords, M, F, sc, ss,
                       w16, h16, lut, h, hq, hs, ng);
  else
    hipLaunchKernelGGL((ks3_spine_kernel<G, false>), grid, dim3(256), 0, st, coords, M, F, sc, ss,
                       w16, h16, lut, h, hq, hs, ng);
}

template <int G>
static void launch_fused(bool vec, dim3 grid, hipStream_t st, const float *acc, int64_t M,
                         int64_t F, const int8_t *sc, const uint16_t *ss, const uint16_t *w16,
                         const uint16_t *h16, const int8_t *lut, int8_t *hq, uint16_t *hs,
                         int64_t ng) {
  if (vec)
    hipLaunchKernelGGL((ks3_spine_fused_kernel<G, true>), grid, dim3(256), 0, st, acc, M, F, sc,
                       ss, w16, h16, lut, hq, hs, ng);
  else
    hipLaunchKernelGGL((ks3_spine_fused_kernel<G, false>), grid, dim3(256), 0, st, acc, M, F, sc,
                       ss, w16, h16, lut, hq, hs, ng);
}

static int64_t vjp_row_blocks(int64_t M) { return cdiv(M, kVjpTile); }

}  // namespace ksd

using namespace ksd;

static int spine_checks(const char *who, const void *in, int64_t M, int64_t F, const int8_t *spine_codes,
                        const uint16_t *spine_scale, const uint16_t *warp_scale,
                        const uint16_t *warp_shift, const int8_t *tanh_lut, int group) {
  if (M < 0 || F < 0) return fail(KSD_EINVAL, "%s: negative shape (%lld, %lld)", who, (long long)M, (long long)F);
  if (!valid_group(group)) return fail(KSD_EINVAL, "%s: group must be 32, 64 or 128", who);
  if (!in || !spine_codes || !spine_scale || !warp_scale || !warp_shift || !tanh_lut)
    return fail(KSD_EINVAL, "%s: null input pointer", who);
  if (((uintptr_t)tanh_lut & 3) != 0) return fail(KSD_EINVAL, "%s: tanh_lut must be 4-byte aligned", who);
  if (cdiv(M, kSpineRows) > 0x7fffffff) return fail(KSD_EINVAL, "%s: M too large", who);
  return KSD_OK;
}

extern "C" int ksd_ks3_spine_fwd(const uint16_t *coords, int64_t M, int64_t F,
                                 const int8_t *spine_codes, const uint16_t *spine_scale,
                                 const uint16_t *warp_scale, const uint16_t *warp_shift,
                                 const int8_t *tanh_lut, int group, float *h, int8_t *h_codes,
                                 uint16_t *h_scales, void *stream) {
  int rc = spine_checks("ks3_spine_fwd", coords, M, F, spine_codes, spine_scale, warp_scale,
                        warp_shift, tanh_lut, group);
  if (rc) return rc;
  if ((h_codes == nullptr) != (h_scales == nullptr))
    return fail(KSD_EINVAL, "ks3_spine_fwd: h_codes and h_scales go together");
  if (!h && !h_codes) return fail(KSD_EINVAL, "ks3_spine_fwd: no output requested");
  if (M == 0 || F == 0) return KSD_OK;
  const bool vec = (F & 3) == 0 && ((uintptr_t)coords & 7) == 0 && ((uintptr_t)h & 15) == 0 &&
                   ((uintptr_t)h_codes & 3) == 0;
  const int64_t ng = cdiv(F, group);
  dim3 grid((unsigned)cdiv(F, 128), (unsigned)cdiv(M, kSpineRows));
  hipStream_t st = (hipStream_t)stream;
#define KSD_SPINE_ARGS vec, grid, st, coords, M, F, spine_codes, spine_scale, warp_scale, warp_shift, \
    tanh_lut, h, h_codes, h_scales, ng
  switch (group) {
    case 32: launch_spine<32>(KSD_SPINE_ARGS); break;
    case 64: launch_spine<64>(KSD_SPINE_ARGS); break;
    default: launch_spine<128>(KSD_SPINE_ARGS); break;
  }
#undef KSD_SPINE_ARGS
  return check_launch("ks3_spine_fwd");
}

extern "C" int ksd_ks3_spine_fused(const float *acc, int64_t M, int64_t F,
                                   const int8_t *spine_codes, const uint16_t *spine_scale,
                                   const uint16_t *warp_scale, const uint16_t *warp_shift,
                                   const int8_t *tanh_lut, int group, int8_t *h_codes,
                                   uint16_t *h_scales, void *stream) {
  int rc = spine_checks("ks3_spine_fused", acc, M, F, spine_codes, spine_scale, warp_scale,
                        warp_shift, tanh_lut, group);
  if (rc) return rc;
  if (!h_codes || !h_scales) return fail(KSD_EINVAL, "ks3_spine_fused: null output pointer");
  if (M == 0 || F == 0) return KSD_OK;
  const bool vec = (F & 3) == 0 && ((uintptr_t)acc & 15) == 0 && ((uintptr_t)h_codes & 3) == 0;
  const int64_t ng = cdiv(F, group);
  dim3 grid((unsigned)cdiv(F, 128), (unsigned)cdiv(M, kSpineRows));
  hipStream_t st = (hipStream_t)stream;
#define KSD_FUSED_ARGS vec, grid, st, acc, M, F, spine_codes, spine_scale, warp_scale, warp_shift, \
    tanh_lut, h_codes, h_scales, ng
  switch (group) {
    case 32: launch_fused<32>(KSD_FUSED_ARGS); break;
    case 64: launch_fused<64>(KSD_FUSED_ARGS); break;
    default: launch_fused<128>(KSD_FUSED_ARGS); break;
  }
#undef KSD_FUSED_ARGS
  return check_launch("ks3_spine_fused");
}

extern "C" int ksd_ks3_vjp_row_blocks(int64_t M, int64_t *n_row_blocks) {
  if (M < 0 || !n_row_blocks) return fail(KSD_EINVAL, "ks3_vjp_row_blocks: bad arguments");
  *n_row_blocks = vjp_row_blocks(M);
  return KSD_OK;
}

extern "C" int ksd_ks3_vjp(const uint16_t *value, const uint16_t *coords, int64_t M, int64_t F,
                           const int8_t *spine_codes, const uint16_t *spine_scale,
                           const uint16_t *warp_scale, const uint16_t *warp_shift, int group,
                           uint16_t *dc, int8_t *dc_codes, uint16_t *dc_scales, int8_t *dct_codes,
                           uint16_t *dct_scales, float *partials, int64_t n_row_blocks, void *stream) {
  if (M < 0 || F < 0) return fail(KSD_EINVAL, "ks3_vjp: negative shape (%lld, %lld)",
                                  (long long)M, (long long)F);
  if (!valid_group(group)) return fail(KSD_EINVAL, "ks3_vjp: group must be 32, 64 or 128");
  if (!value || !coords || !spine_codes || !spine_scale || !warp_scale || !warp_shift || !partials)
    return fail(KSD_EINVAL, "ks3_vjp: null input or partials pointer");
  if ((dc_codes == nullptr) != (dc_scales == nullptr) || (dct_codes == nullptr) != (dct_scales == nullptr))
    return fail(KSD_EINVAL, "ks3_vjp: codes and scales outputs go together");
  if (M == 0 || F == 0) return KSD_OK;
  if (n_row_blocks != vjp_row_blocks(M))
    return fail(KSD_EINVAL, "ks3_vjp: partials must hold ksd_ks3_vjp_row_blocks(M)=%lld row blocks, got %lld",
                (long long)vjp_row_blocks(M), (long long)n_row_blocks);
  if ((F & 1) == 0 && ((((uintptr_t)value | (uintptr_t)coords | (uintptr_t)dc) & 3) != 0 ||
                       ((uintptr_t)dc_codes & 1) != 0))
    return fail(KSD_EINVAL, "ks3_vjp: value/coords/dc must be 4-byte and dc_codes 2-byte aligned");
  if ((M & 15) == 0 && ((uintptr_t)dct_codes & 15) != 0)
    return fail(KSD_EINVAL, "ks3_vjp: dct_codes must be 16-byte aligned");
  if ((int64_t)kVjpTile * F * 2 > 0x7fffffff || (int64_t)kVjpTile * M > 0x7fffffff)
    return fail(KSD_EINVAL, "ks3_vjp: F or M too large for 32-bit tile offsets");
  dim3 grid((unsigned)cdiv(F, kVjpTile), (unsigned)n_row_blocks);
  hipStream_t st = (hipStream_t)stream;
  const bool vec = (F & 1) == 0;
#define KSD_VJP_ARGS value, coords, M, F, spine_codes, spine_scale, warp_scale, warp_shift, dc, \
    dc_codes, dc_scales, dct_codes, dct_scales, partials
#define KSD_VJP_LAUNCH(G)                                                                      \
  if (vec) hipLaunchKernelGGL((ks3_vjp_kernel<G, true>), grid, dim3(256), 0, st, KSD_VJP_ARGS); \
  else hipLaunchKernelGGL((ks3_vjp_kernel<G, false>), grid, dim3(256), 0, st, KSD_VJP_ARGS);
  switch (group) {
    case 32: KSD_VJP_LAUNCH(32) break;
    case 64: KSD_VJP_LAUNCH(64) break;
    default: KSD_VJP_LAUNCH(128) break;
  }
#undef KSD_VJP_LAUNCH
#undef KSD_VJP_ARGS
  return check_launch("ks3_vjp");
}

extern "C" int ksd_ks3_vjp_finalize(const float *partials, int64_t n_row_blocks, int64_t F,
                                    const float *warp_scale_raw, const float *warp_shift_raw,
                                    float *sums, uint16_t *dcoeff, uint16_t *dscale, uint16_t *dshift,
                                    void *stream) {
  if (F < 0 || n_row_blocks < 0) return fail(KSD_EINVAL, "ks3_vjp_finalize: negative shape");
  if (!partials || !warp_scale_raw || !warp_shift_raw || !dcoeff || !dscale || !dshift)
    return fail(KSD_EINVAL, "ks3_vjp_finalize: null pointer");
  if (F == 0) return KSD_OK;
  hipLaunchKernelGGL(ks3_vjp_finalize_kernel, dim3((unsigned)cdiv(F, 256)), dim3(256), 0,
                     (hipStream_t)stream, partials, n_row_blocks, F, warp_scale_raw, warp_shift_raw,
                     sums, dcoeff, dscale, dshift);
  return check_launch("ks3_vjp_finalize");
}

extern "C" int ksd_ks3_tanh16(const uint16_t *x, int64_t n, uint16_t *y, void *stream) {
  if (n < 0 || (n > 0 && (!x || !y))) return fail(KSD_EINVAL, "ks3_tanh16: bad arguments");
  if (n == 0) return KSD_OK;
  hipLaunchKernelGGL(ks3_tanh16_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                     (hipStream_t)stream, x, n, y);
  return check_launch("ks3_tanh16");
}
