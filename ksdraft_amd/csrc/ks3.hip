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

// The warp step tq * (4/127). Composed (ks3_int8.py:211): a torch fp16 tensor times a
// Python float is evaluated in fp32 with the constant in fp32. Fused (ks3_triton.py:59):
// Triton keeps a Python-float scalar out of type promotion (triton/language/semantic.py,
// computation_type_impl), so the product is fp16 arithmetic with the constant fp16(4/127),
// and its compiled form contracts it with the add of the shift into one v_fma_f16.
constexpr float kTq16Step = (float)(4.0 / 127.0);
constexpr float kTq16StepFused = 0.031494140625f;  // fp16(4/127) = 2064 * 2^-16

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

// The chart part of _spine_features 'int8' mode, rank 1 (ks3_int8.py:209-225), and of the
// fused kernel's spine (ks3_triton.py:52-70): for the LUT index ti of a coordinate, tq =
// LUT[ti], the warp w(tq) and zq = LUT[index(w)], then the two integer Horner sums. Every
// step depends on the chart and ti alone, so the kernels tabulate it per chart over the 256
// indices: the composed contract as its fp16 increment fp16(fp16(trunc(sum / 64)) * ps)
// (:226-227), the fused one as its fp32 increment sum * (ps / 64) (ks3_triton.py:70).
template <bool FUSED>
__device__ __forceinline__ int spine_sum(int ti, const SpineCol &c, const int8_t *lut) {
  const int tq = lut_at(lut, ti);
  float w;
  if constexpr (FUSED) {
    // ks3_triton.py:59 as Triton compiles it for gfx950: the fp16 product and the add of
    // the shift are one v_fma_f16 (one rounding), then an fp16 multiply by the scale
    const _Float16 t16 = __builtin_fmaf16((_Float16)tq, (_Float16)kTq16StepFused, (_Float16)c.sh);
    w = (float)((_Float16)c.sc * t16);
  } else {
    // ks3_int8.py:211: torch's fp16 ops, each evaluated in fp32 and rounded to fp16
    w = f16_round(f16_round((float)tq * kTq16Step) + c.sh);
    w = f16_round(c.sc * w);
  }
  const int zq = lut_at(lut, FUSED ? (int)rintf(fminf(fmaxf(w, -kLutDomain), kLutDomain) * kLutScale)
                                   : lut_index(w));
  int poly = c.a64;
  poly = round_div127(poly * tq * 4) + c.b64;
  poly = round_div127(poly * tq * 4) + c.c2_64;
  poly = round_div127(poly * tq * 4) + c.c0_64;
  int wp = c.c5x4_64;
  wp = round_div127(wp * zq) + c.c4x2_64;
  wp = round_div127(wp * zq) - c.c5x3_64;
  wp = round_div127(wp * zq) - c.c4_64;
  return poly + wp;
}

// Table builder: block = one chart, thread = LUT index ti + 128 (0..255). Composed: fp16
// bits of the increment; fused: fp32 bits.
template <bool FUSED>
__global__ void __launch_bounds__(256) ks3_spine_table_kernel(
    const int8_t *__restrict__ spine_codes, const uint16_t *__restrict__ spine_scale,
    const uint16_t *__restrict__ sc16, const uint16_t *__restrict__ sh16,
    const int8_t *__restrict__ tanh_lut, void *__restrict__ table) {
  __shared__ int8_t lut[256];
  if (threadIdx.x < 64) ((uint32_t *)lut)[threadIdx.x] = ((const uint32_t *)tanh_lut)[threadIdx.x];
  __syncthreads();
  const int64_t f = blockIdx.x;
  const SpineCol c = load_spine_col(spine_codes, spine_scale, sc16, sh16, f, true);
  const int sum = spine_sum<FUSED>((int)threadIdx.x - 128, c, lut);
  if constexpr (FUSED) {
    ((float *)table)[f * 256 + threadIdx.x] = (float)sum * (c.ps / 64.0f);
  } else {
    const int td = sum / 64;  // torch.div(..., rounding_mode="trunc")
    ((uint16_t *)table)[f * 256 + threadIdx.x] = f16_bits(f16_round((float)td) * c.ps);
  }
}

// _lut_index of an fp16 coordinate x (ks3_int8.py:69-72, composed contract). x / 4 is
// exact in fp16 unless |x| < 2^-12, where either way the index is 0, so the fp16 rounding
// of x * 0.25 is skipped; clamping an fp16 value to the fp16 bounds +-fp16(3.2) equals
// torch's clamp to +-3.2 followed by the fp16 rounding.
__device__ __forceinline__ int lut_index_x(float x) {
  constexpr float kDom16 = 3.19921875f;  // fp16(3.2)
  const float c = __builtin_amdgcn_fmed3f(x * 0.25f, -kDom16, kDom16);
  return (int)rintf(f16_round(c * kLutScale));
}

// rint(h / pre) clamped to [0, 127] for the rank-1 ReLU^2 codes (ks3_int8.py:232): the
// reciprocal multiply of codes_rcp (within 2^-15 of the quotient for |p| <= 128), the
// IEEE division when p lies within 2^-14 of a half-integer. NaN gives 0 as fmax/fmin do.
__device__ __forceinline__ float relu2_code(float h, float pre) {
  const float p = h * __builtin_amdgcn_rcpf(pre);
  float t = rintf(p);
  if (fabsf(fabsf(p - t) - 0.5f) < 0x1p-14f) t = rintf(h / pre);
  return fmaxf(fminf(fmaxf(t, -127.0f), 127.0f), 0.0f);
}

// Max over the 32 lanes of each half-wave (u32 patterns): DPP within 16-lane rows, then
// a ds_swizzle exchange of lanes i and i ^ 16.
__device__ __forceinline__ uint32_t group_max32_u32(uint32_t v) {
  v = group_max_u32<16>(v);
  return max(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401f));
}
template <int L>
__device__ __forceinline__ uint32_t lane_group_max(uint32_t v) {
  if constexpr (L == 32) return group_max32_u32(v);
  else return group_max_u32<L>(v);
}

// Spine kernels: block = 512 threads = 16 rows x 32 lanes; a lane owns 4 consecutive
// charts of the block's 128-chart segment (blockIdx.x), so a G-chart group is G/4 lanes of
// one half-wave. Rows [blockIdx.y * kSpineRows, +kSpineRows), 2 per lane per iteration
// with both rows' loads issued first. The segment's increment table (128 charts x 256
// indices) is staged in LDS with a pitch of 129 words (fp16 table) / 257 words (fp32):
// lanes reading the same index of different charts then fall in different banks.
constexpr int kSpineRows = 512;
constexpr int kSpineThreads = 512;

template <bool FUSED>
struct SpineTab {
  static constexpr int kPitch = FUSED ? 257 : 129;  // 32-bit words per chart
  __device__ static void stage(uint32_t *tab, const void *table, int64_t c0, int64_t F) {
    constexpr int WPC = FUSED ? 256 : 128;           // words per chart in global memory
    const uint32_t *src = (const uint32_t *)table;
    for (int i = threadIdx.x; i < 128 * WPC / 4; i += kSpineThreads) {
      const int ch = i / (WPC / 4), w4 = i % (WPC / 4);
      uint4 v = make_uint4(0, 0, 0, 0);
      if (c0 + ch < F) v = *(const uint4 *)(src + (c0 + ch) * WPC + w4 * 4);
      uint32_t *d = tab + ch * kPitch + w4 * 4;
      d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
    }
  }
  __device__ static float inc(const uint32_t *tab, int ch, int idx) {
    if constexpr (FUSED) return __builtin_bit_cast(float, tab[ch * kPitch + idx]);
    else return f16_to_f32(((const uint16_t *)tab)[ch * (2 * kPitch) + idx]);
  }
};

// LUT byte offsets (2 * (ti + 128)) of two fp16 coordinates packed in a word, on packed
// fp16 (the composed contract's _lut_index, ks3_int8.py:69-72): x * 0.25 (exact, and where
// it is not, |x| < 2^-12, the index is 0 either way), the clamp to +-fp16(3.2) (equal to
// torch's fp32 clamp followed by fp16 rounding), the fp16 product with 127/3.2 (exact in
// fp32, so rounding once to fp16 equals torch's two roundings), then + 1.5 * 2^10, which
// rounds to an integer (ties to even) and leaves 0x6600 + ti in the bits (|ti| <= 127).
__device__ __forceinline__ void lut_offsets2(uint32_t xw, uint32_t &o0, uint32_t &o1) {
  const h2 kQ = {(_Float16)0.25f, (_Float16)0.25f};
  const h2 kLo = {(_Float16)-3.19921875f, (_Float16)-3.19921875f};
  const h2 kHi = {(_Float16)3.19921875f, (_Float16)3.19921875f};
  const h2 kS = {(_Float16)39.6875f, (_Float16)39.6875f};
  const h2 kM = {(_Float16)1536.0f, (_Float16)1536.0f};
  h2 c = __builtin_bit_cast(h2, xw) * kQ;
  c = __builtin_elementwise_min(__builtin_elementwise_max(c, kLo), kHi);
  const uint32_t b = __builtin_bit_cast(uint32_t, c * kS + kM);
  o0 = ((b & 0xffffu) - 0x6580u) * 2u;
  o1 = ((b >> 16) - 0x6580u) * 2u;
}

// fp16(clamp(h / 127, 2^-24, 65504)) for a finite or NaN h >= 0 (group_scale of one
// element: the div127 correction needs no infinity guard, and the clamp propagates NaN).
__device__ __forceinline__ float scale_of_finite(float h) {
  constexpr float r = 1.0f / 127.0f;
  const float q0 = h * r;
  const float q = fmaf(fmaf(-q0, 127.0f, h), r, q0);
  return f16_round(__builtin_elementwise_minimum(__builtin_elementwise_maximum(q, kScaleMin), kScaleMax));
}

// Composed contract (ks3_int8.py:205-234 + quantize_last_dim(h, G)): x is the fp16
// coordinate; h = relu(x + inc[ti]); the rank-1 ReLU^2 requantization pre = fp16 scale of
// |h|, code q = rint(h / pre) in [0, 127], feature fp16(q * q) * pre^2; then the feature's
// per-group quantization. Per iteration a lane takes 2 rows x 4 charts in phases (loads,
// LUT offsets, the 8 table reads, the arithmetic), with one fallback branch for the rare
// near-tie ReLU^2 codes; codes and scales leave through buffer stores whose offsets for
// rows past the block's end or charts past F lie past num_records.
template <int G, bool VEC>
__global__ void __launch_bounds__(kSpineThreads) ks3_spine_kernel(
    const uint16_t *__restrict__ coords, int64_t M, int64_t F, const void *__restrict__ table,
    float *__restrict__ h_out, int8_t *__restrict__ hq, uint16_t *__restrict__ hs, int64_t n_groups) {
  using Tab = SpineTab<false>;
  __shared__ uint32_t tab[128 * Tab::kPitch];
  const int64_t c0 = (int64_t)blockIdx.x * 128;
  Tab::stage(tab, table, c0, F);
  __syncthreads();
  const int lane = threadIdx.x & 31;
  const int rsub = threadIdx.x >> 5;
  const int64_t col0 = c0 + lane * 4;
  const bool cok = col0 < F;
  const bool seg_full = c0 + 128 <= F;             // block-uniform: no chart past F
  const int64_t colc = cok ? col0 : 0;             // a valid column for every lane
  const uint32_t tab_lane = (uint32_t)(uintptr_t)(tab) + (uint32_t)(lane * 4) * (4 * Tab::kPitch);
  const int64_t row_end = min(M, (int64_t)(blockIdx.y + 1) * kSpineRows);
  const int64_t rbase = (int64_t)blockIdx.y * kSpineRows, nrows = row_end - rbase;
  const int64_t rfirst = rbase + rsub;
  // the two rows (r0, r0 + 16) of an iteration as packed fp16 words: 4 charts each
  auto raw2 = [&](int64_t r0, uint2 (&w)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint16_t *src = coords + min(r0 + 16 * u, M - 1) * F + colc;
      if (VEC) {
        w[u] = *(const uint2 *)src;
      } else {
        uint32_t e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = col0 + j < F ? src[j] : 0u;
        w[u] = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
      }
    }
  };
  auto body = [&](int64_t r0, const uint2 (&w)[2]) __attribute__((always_inline)) {
    uint32_t off[2][4];
    float x[2][4], inc[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      lut_offsets2(w[u].x, off[u][0], off[u][1]);
      lut_offsets2(w[u].y, off[u][2], off[u][3]);
      x[u][0] = f16_to_f32((uint16_t)w[u].x);
      x[u][1] = f16_to_f32((uint16_t)(w[u].x >> 16));
      x[u][2] = f16_to_f32((uint16_t)w[u].y);
      x[u][3] = f16_to_f32((uint16_t)(w[u].y >> 16));
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        typedef __attribute__((address_space(3))) const uint16_t lds_u16;
        inc[u][j] = f16_to_f32(*(lds_u16 *)(uintptr_t)(tab_lane + j * (4 * Tab::kPitch) + off[u][j]));
      }
    float v[2][4], pre[2][4], h[2][4];
    float near = 1.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // relu (NaN-propagating max; -0 becomes +0, which leaves every output unchanged)
        const float t = __builtin_elementwise_maximum(x[u][j] + inc[u][j], 0.0f);
        v[u][j] = t;
        pre[u][j] = scale_of_finite(t);  // amax over the rank dim (one element), :230-231
        const float p = t * __builtin_amdgcn_rcpf(pre[u][j]);
        const float r = rintf(p);
        near = fminf(near, fabsf(fabsf(p - r) - 0.5f));
        h[u][j] = r;
      }
    if (near < 0x1p-14f) {  // some quotient within 2^-14 of a half-integer: divide
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) h[u][j] = rintf(v[u][j] / pre[u][j]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // q = clamp(rint(h / pre), 0, 127); a NaN q leaves the feature NaN via pre
        const float q = __builtin_amdgcn_fmed3f(h[u][j], 0.0f, 127.0f);
        const float f = f16_round(q * q) * (pre[u][j] * pre[u][j]);
        h[u][j] = seg_full || (VEC ? cok : col0 + j < F) ? f : 0.0f;
      }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t row = r0 + 16 * u;
      const bool rok = row < row_end;
      if (h_out && rok) {
        float *dst = h_out + row * F + col0;
        if (VEC && cok) {
          *(float4 *)dst = make_float4(h[u][0], h[u][1], h[u][2], h[u][3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (col0 + j < F) dst[j] = h[u][j];
        }
      }
      if (hq) {
        // quantize_last_dim(h, G): one group = G/4 lanes of a half-wave
        const uint32_t am = lane_group_max<G / 4>(__builtin_bit_cast(uint32_t, abs_max<4>(h[u])));
        const float s = group_scale(__builtin_bit_cast(float, am));
        uint32_t wq;
        codes_rcp_packed<4>(h[u], s, &wq);
        // block-uniform descriptors (a per-lane base makes the compiler loop over a wave's
        // distinct descriptors around every store); the lane's row goes into the offset
        const int64_t lr = row - rbase;
        const bool lead = rok && cok && (lane & (G / 4 - 1)) == 0;
        __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rsrc(hs + rbase * n_groups, 2 * nrows * n_groups),
                                              lead ? (uint32_t)(lr * n_groups + col0 / G) * 2 : kOob, 0, 0);
        if (VEC) {
          __builtin_amdgcn_raw_buffer_store_b32(wq, rsrc(hq + rbase * F, nrows * F),
                                                rok && cok ? (uint32_t)(lr * F + col0) : kOob, 0, 0);
        } else if (rok) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (col0 + j < F) hq[row * F + col0 + j] = (int8_t)(wq >> (8 * j));
        }
      }
    }
  };
  // two row pairs in flight: the pair after next is loaded (from clamped valid rows) before
  // this pair's arithmetic, into the buffer the previous pair just released; a fixed trip
  // count, rows past the block's end only having their stores masked
  uint2 wa[2], wb[2];
  raw2(rfirst, wa);
  raw2(rfirst + 32, wb);
#pragma unroll 1
  for (int it = 0; it < kSpineRows / 64; ++it) {
    const int64_t r0 = rfirst + 64 * it;
    const uint2 ca[2] = {wa[0], wa[1]};
    raw2(r0 + 64, wa);
    body(r0, ca);
    const uint2 cb[2] = {wb[0], wb[1]};
    raw2(r0 + 96, wb);
    body(r0 + 32, cb);
  }
}

// The fused-kernel contract of project_fused / _fused_gemm_spine, 'int8' mode
// (ks3_triton.py:47-75, 137-156). It differs from the composed one: x is the fp32 GEMM
// accumulator clamped to +-65504 (no fp16 materialisation); LUT indices are computed in
// fp32; the Horner sum is scaled by ps/64 in fp32 without truncation; the ReLU^2 pre-scale
// is the amax of |h| (before ReLU) over the row's G-chart group; the squared codes are
// exact; and the result is requantized per group a second time. Same block layout, row
// prefetch and phase order as ks3_spine_kernel.
template <int G, bool VEC>
__global__ void __launch_bounds__(kSpineThreads) ks3_spine_fused_kernel(
    const float *__restrict__ acc, int64_t M, int64_t F, const void *__restrict__ table,
    int8_t *__restrict__ hq, uint16_t *__restrict__ hs, int64_t n_groups) {
  using Tab = SpineTab<true>;
  __shared__ uint32_t tab[128 * Tab::kPitch];
  const int64_t c0 = (int64_t)blockIdx.x * 128;
  Tab::stage(tab, table, c0, F);
  __syncthreads();
  const int lane = threadIdx.x & 31;
  const int rsub = threadIdx.x >> 5;
  const int64_t col0 = c0 + lane * 4;
  const bool cok = col0 < F;
  const bool seg_full = c0 + 128 <= F;
  const int64_t colc = cok ? col0 : 0;
  const uint32_t tab_lane = (uint32_t)(uintptr_t)(tab) + (uint32_t)(lane * 4) * (4 * Tab::kPitch);
  const int64_t row_end = min(M, (int64_t)(blockIdx.y + 1) * kSpineRows);
  const int64_t rbase = (int64_t)blockIdx.y * kSpineRows, nrows = row_end - rbase;
  const int64_t rfirst = rbase + rsub;
  auto raw2 = [&](int64_t r0, float4 (&w)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float *src = acc + min(r0 + 16 * u, M - 1) * F + colc;
      if (VEC) {
        w[u] = *(const float4 *)src;
      } else {
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = col0 + j < F ? src[j] : 0.0f;
        w[u] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
  };
  auto body = [&](int64_t r0, const float4 (&w)[2]) __attribute__((always_inline)) {
    float xc[2][4], h[2][4];
    uint32_t off[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float xs[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xc[u][j] = fminf(fmaxf(xs[j], -kScaleMax), kScaleMax);  // as the reference clamp (a NaN -> -65504)
        off[u][j] = (uint32_t)(min(max(lut_index_f32(xc[u][j] * 0.25f) + 128, 0), 255)) * 4u;
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        typedef __attribute__((address_space(3))) const float lds_f32;
        const float inc = *(lds_f32 *)(uintptr_t)(tab_lane + j * (4 * Tab::kPitch) + off[u][j]);
        h[u][j] = seg_full || col0 + j < F ? xc[u][j] + inc : 0.0f;
      }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t row = r0 + 16 * u;
      const bool rok = row < row_end;
      const uint32_t am = lane_group_max<G / 4>(__builtin_bit_cast(uint32_t, abs_max<4>(h[u])));
      const float pre = group_scale(__builtin_bit_cast(float, am));
      const float rp = __builtin_amdgcn_rcpf(pre);
      float t[4];
      float near = 1.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p = h[u][j] * rp;
        t[j] = rintf(p);
        near = fminf(near, fabsf(fabsf(p - t[j]) - 0.5f));
      }
      if (near < 0x1p-14f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = rintf(h[u][j] / pre);
      }
      float f[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float q = __builtin_amdgcn_fmed3f(t[j], 0.0f, 127.0f);  // NaN q: NaN via pre
        f[j] = (q * q) * (pre * pre);
      }
      const uint32_t hm = lane_group_max<G / 4>(__builtin_bit_cast(uint32_t, abs_max<4>(f)));
      const float s = group_scale(__builtin_bit_cast(float, hm));
      uint32_t wq;
      codes_rcp_packed<4>(f, s, &wq);
      const int64_t lr = row - rbase;  // block-uniform descriptors, as in ks3_spine_kernel
      const bool lead = rok && cok && (lane & (G / 4 - 1)) == 0;
      __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rsrc(hs + rbase * n_groups, 2 * nrows * n_groups),
                                            lead ? (uint32_t)(lr * n_groups + col0 / G) * 2 : kOob, 0, 0);
      if (VEC) {
        __builtin_amdgcn_raw_buffer_store_b32(wq, rsrc(hq + rbase * F, nrows * F),
                                              rok && cok ? (uint32_t)(lr * F + col0) : kOob, 0, 0);
      } else if (rok) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (col0 + j < F) hq[row * F + col0 + j] = (int8_t)(wq >> (8 * j));
      }
    }
  };
  float4 wa[2], wb[2];
  raw2(rfirst, wa);
  raw2(rfirst + 32, wb);
#pragma unroll 1
  for (int it = 0; it < kSpineRows / 64; ++it) {
    const int64_t r0 = rfirst + 64 * it;
    const float4 ca[2] = {wa[0], wa[1]};
    raw2(r0 + 64, wa);
    body(r0, ca);
    const float4 cb[2] = {wb[0], wb[1]};
    raw2(r0 + 96, wb);
    body(r0 + 32, cb);
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

// vjp_pair over N rows in phases: the N first tanh lookups, then the N warp lookups, then
// the arithmetic of each row, so the LDS reads of different rows overlap. Same op-by-op
// fp16 arithmetic as vjp_pair.
template <int N>
__device__ __forceinline__ void vjp_rows(const h2 *v, const h2 *x, const VjpCols &c,
                                         const uint16_t *tab, float (*acc)[2], h2 *dc) {
  const h2 one = bc((_Float16)1.0f);
  h2 t[N], tps[N], z[N];
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = tanh2(x[i] * bc((_Float16)0.25f), tab);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    t[i] = bc((_Float16)4.0f) * t[i];
    tps[i] = t[i] + c.sh;
    z[i] = tanh2(c.sc * tps[i], tab);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const h2 ti = t[i], zi = z[i];
    h2 spine = c.cubic * ti + c.quad;
    spine = spine * ti + c.c2;
    spine = spine * ti + c.c0;
    h2 warped = c.c5x4 * zi + c.c4x2;
    warped = warped * zi - c.c5x3;
    warped = warped * zi - c.c4;
    h2 pre = x[i] + spine;
    pre = pre + warped;
    pre = pre < bc((_Float16)0.0f) ? bc((_Float16)0.0f) : pre;  // torch.relu: keeps -0 and NaN
    const h2 dpre = (v[i] * bc((_Float16)2.0f)) * pre;
    h2 dpoly = c.cubic3 * ti + c.quad2;
    dpoly = dpoly * ti + c.c2;
    h2 dwarp = c.c5x12 * zi + c.c4x4;
    dwarp = dwarp * zi - c.c5x3;
    const h2 z2 = zi * zi;
    const h2 dz = dwarp * (one - z2);
    const h2 t2 = ti * ti;
    const h2 dmean = (dpre * (dpoly + dz * c.sc)) * (one - t2 * bc((_Float16)0.0625f));
    const h2 t3 = t2 * ti;
    const h2 z3 = z2 * zi;
    const h2 t3x2 = bc((_Float16)2.0f) * t3;
    const h2 t2x3 = bc((_Float16)3.0f) * t2;
    const h2 dpdz = dpre * dz;
    const h2 terms[8] = {
        dpre * ((t3x2 - t2x3) + one),
        dpre * (t2x3 - t3x2),
        dpre * ((t3 - bc((_Float16)2.0f) * t2) + ti),
        dpre * (t3 - t2),
        dpre * (bc((_Float16)2.0f) * z2 - one),
        dpre * (bc((_Float16)4.0f) * z3 - bc((_Float16)3.0f) * zi),
        dpdz * tps[i],
        dpdz * c.sc,
    };
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      acc[k][0] = add_lo(acc[k][0], terms[k]);
      acc[k][1] = add_hi(acc[k][1], terms[k]);
    }
    dc[i] = v[i] + dmean;
  }
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

// Max of packed u16 pairs (fp16 magnitudes: the NaN-propagating order) over aligned groups
// of L lanes (2..64): DPP within 16-lane rows, ds_swizzle across a half-wave, and the two
// half-waves' lane 0 / lane 32 values for the whole wave (then wave-uniform).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}
template <int L>
__device__ __forceinline__ uint32_t group_max_pk16(uint32_t v) {
  if constexpr (L >= 2) v = pk_max_u16(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  if constexpr (L >= 4) v = pk_max_u16(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  if constexpr (L >= 8) v = pk_max_u16(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  if constexpr (L >= 16) v = pk_max_u16(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  if constexpr (L >= 32) v = pk_max_u16(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401f));
  if constexpr (L >= 64)
    v = pk_max_u16((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 32));
  return v;
}

// Row tiles (128 rows) per VJP block: the tanh table is staged once per block and the
// eight column sums are reduced once per block (one partial row per kVjpRowsPerBlock rows).
constexpr int kVjpTilesPerBlock = 4;
constexpr int kVjpRowsPerBlock = kVjpTile * kVjpTilesPerBlock;

// Block: 256 threads (4 waves) on 128 columns (blockIdx.x) and kVjpTilesPerBlock row tiles
// of 128 rows (blockIdx.y). In a tile, lane l owns columns 2l and 2l+1 of the 32 rows
// wave*32 + i; a register holds one row at both columns. VEC: F is even, so a lane's two
// columns are both valid or both past F.
template <int G, bool VEC>
__global__ void __launch_bounds__(256) ks3_vjp_kernel(
    const uint16_t *__restrict__ value, const uint16_t *__restrict__ coords, int64_t M, int64_t F,
    const int8_t *__restrict__ spine_codes, const uint16_t *__restrict__ spine_scale,
    const uint16_t *__restrict__ sc16, const uint16_t *__restrict__ sh16,
    uint16_t *__restrict__ dc_out, int8_t *__restrict__ dcq, uint16_t *__restrict__ dcs,
    int8_t *__restrict__ dctq, uint16_t *__restrict__ dcts, float *__restrict__ partials) {
  __shared__ __attribute__((aligned(16))) uint32_t tabw[KSD_TANH16_WORDS];
  __shared__ uint32_t colmax[4][kVjpTile / 2];  // packed fp16 column maxima per wave
  const uint16_t *tab = (const uint16_t *)tabw;
  for (int i = threadIdx.x; i < KSD_TANH16_WORDS / 4; i += 256)
    ((uint4 *)tabw)[i] = ((const uint4 *)kTanh16)[i];
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
  const uint32_t rstride2 = (uint32_t)(F * 2);
  __syncthreads();

  for (int tt = 0; tt < kVjpTilesPerBlock; ++tt) {
    const int64_t tr0 = (int64_t)blockIdx.y * kVjpRowsPerBlock + (int64_t)tt * kVjpTile;
    if (tr0 >= M) break;                                 // block-uniform
    const int r0 = wave * 32;                            // first tile row of this wave
    const int64_t grow0 = tr0 + r0;                      // global row of this wave's first row
    const auto rv = rows_rsrc(value, grow0, 32, M, F);
    const auto rx = rows_rsrc(coords, grow0, 32, M, F);

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
      for (int q = 0; q < 16; q += 4) {
        __builtin_amdgcn_sched_barrier(0);
        vjp_rows<4>(va + q, xa + q, cc, tab, acc, dc + half * 16 + q);
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
    // G/2 lanes. Two rows are reduced per packed register; codes by reciprocal multiply
    // (codes_rcp_packed's bound), the division redoing two rows with a near-tie quotient.
    if (dcq) {
      const bool writes_scale = (lane & (G / 2 - 1)) == 0 && ok0;
      const uint32_t soff = writes_scale ? (uint32_t)(col0 / G * 2) : kOob;
      const auto rq = rows_rsrc(dcq, grow0, 32, M, F);
      const auto rsc = rows_rsrc(dcs, grow0, 32, M, ngF);
#pragma unroll
      for (int i = 0; i < 32; i += 2) {
        const h2 a0 = habs2(dc[i]), a1 = habs2(dc[i + 1]);
        const h2 m = __builtin_bit_cast(
            h2, group_max_pk16<G / 2>(__builtin_bit_cast(uint32_t, hmax2((h2){a0[0], a1[0]}, (h2){a0[1], a1[1]}))));
        float s[2], f[2][2];
        uint32_t mg[2][2];
        float near = 1.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          s[e] = group_scale((float)m[e]);
          const float r = __builtin_amdgcn_rcpf(s[e]);
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            f[e][c] = (float)dc[i + e][c];
            const float q = __builtin_amdgcn_fmed3f(f[e][c] * r, -127.0f, 127.0f);
            const float mq = q + 12582912.0f;
            near = fminf(near, half_dist(q));
            mg[e][c] = __builtin_bit_cast(uint32_t, mq);
            if (s[e] != s[e]) mg[e][c] = 0;  // NaN group: zero codes
          }
        }
        if (near < 0x1p-14f) {
#pragma unroll
          for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int c = 0; c < 2; ++c) mg[e][c] = (uint8_t)code_of(f[e][c] / s[e]);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const uint32_t ro = (uint32_t)((i + e) * F);
          const uint32_t q0 = mg[e][0] & 0xffu, q1 = mg[e][1] & 0xffu;
          if (VEC) {
            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(q0 | (q1 << 8)), rq, voff1 + ro, 0, 0);
          } else {
            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)q0, rq, voff1 + ro, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)q1, rq, voff1b + ro, 0, 0);
          }
          __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s[e]), rsc, soff + (uint32_t)((i + e) * ngF * 2), 0, 0);
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
        float col[32];
#pragma unroll
        for (int r = 0; r < 32; ++r) col[r] = (float)dc[r][e];
        uint32_t w[8];
        codes_rcp_packed<32>(col, s, w);
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
  float *red = (float *)tabw;  // [4 waves][8 terms][128 cols] = 16 KiB
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
    float sum = red[(0 * 8 + k) * kVjpTile + c];
    sum += red[(1 * 8 + k) * kVjpTile + c];
    sum += red[(2 * 8 + k) * kVjpTile + c];
    sum += red[(3 * 8 + k) * kVjpTile + c];
    partials[((int64_t)blockIdx.y * 8 + k) * F + col] = sum;
  }
}

// Fixed-order sum of the per-block partials, then the reference's fp16 roundings and the
// STE chain to the raw warp parameters (ks3_int8.py:379-395). One thread per (reduction k,
// chart f): eight interleaved accumulators (row block b goes to accumulator b mod 8), added
// pairwise at the end, so the order depends on the row-block count only, not on the device.
__global__ void ks3_vjp_finalize_kernel(const float *__restrict__ partials, int64_t nrb, int64_t F,
                                        const float *__restrict__ raw_scale,
                                        const float *__restrict__ raw_shift, float *__restrict__ sums,
                                        uint16_t *__restrict__ dcoeff, uint16_t *__restrict__ dscale,
                                        uint16_t *__restrict__ dshift) {
  const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int k = blockIdx.y;
  if (f >= F) return;
  const float *p = partials + (int64_t)k * F + f;
  const int64_t step = 8 * F;
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  int64_t b = 0;
  for (; b + 8 <= nrb; b += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = p[(b + j) * step];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += v[j];
  }
  for (int j = 0; b < nrb; ++b, ++j) acc[j] += p[b * step];
  const float a = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  if (sums) sums[k * F + f] = a;
  if (k < 6) {
    dcoeff[f * 6 + k] = f16_bits(a);
  } else if (k == 6) {
    const float sig = 1.0f / (1.0f + expf(-raw_scale[f]));
    dscale[f] = f16_bits(f16_round(a) * sig);
  } else {
    const float th = tanhf(raw_shift[f]);
    dshift[f] = f16_bits(f16_round(f16_round(a) * 0.5f) * (1.0f - th * th));
  }
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
                         int64_t F, const void *table, float *h, int8_t *hq, uint16_t *hs, int64_t ng) {
  if (vec)
    hipLaunchKernelGGL((ks3_spine_kernel<G, true>), grid, dim3(kSpineThreads), 0, st, coords, M, F,
                       table, h, hq, hs, ng);
  else
    hipLaunchKernelGGL((ks3_spine_kernel<G, false>), grid, dim3(kSpineThreads), 0, st, coords, M, F,
                       table, h, hq, hs, ng);
}

template <int G>
static void launch_fused(bool vec, dim3 grid, hipStream_t st, const float *acc, int64_t M,
                         int64_t F, const void *table, int8_t *hq, uint16_t *hs, int64_t ng) {
  if (vec)
    hipLaunchKernelGGL((ks3_spine_fused_kernel<G, true>), grid, dim3(kSpineThreads), 0, st, acc, M,
                       F, table, hq, hs, ng);
  else
    hipLaunchKernelGGL((ks3_spine_fused_kernel<G, false>), grid, dim3(kSpineThreads), 0, st, acc,
                       M, F, table, hq, hs, ng);
}

static int64_t vjp_row_blocks(int64_t M) { return cdiv(M, kVjpRowsPerBlock); }

// ---------------------------------------------------------------- float nonlinear modes
// _spine_features in the 'fp32' and 'fp16' modes (ks3_int8.py:172-203), rank 1, with the
// features requantized along F in the same pass (quantize_last_dim(h), group G). SRC is
// KSD_F16 for the composed path (the coordinates the GEMM epilogue rounded to fp16 and
// clamped) or KSD_F32 for the project_fused contract (the fp32 down-GEMM accumulator,
// clamped to +-65504 here, ks3_triton.py:146). sc / sh are the warp scalars as fp32 values
// (the caller passes the fp32 or fp16 dequantization the path uses).
//   fp32:  t = 4 tanh(x / 4), z = tanh(sc (t + sh)), the Horner cubic and warp in fp32,
//          h = relu(x + (poly + warped) ps)^2, every op rounded to fp32 (tanh: tanhf).
//   fp16:  th = fp16(x / 4), t = fp16(4 tanh(th)), warp = fp16(sc (t + sh)) (two fp32
//          ops), z = fp16(tanh(warp)), the Horner steps as fp16 ops, h = relu(fp16(x +
//          (poly + warped) ps)) and fp16(h h). tanh of an fp16 value rounded to fp16 comes
//          from the kTanh16 table (staged in LDS); fp16(4 tanh(th)) equals 4 table(th)
//          for |th| >= 2^-12 (where the table value is a normal fp16, so the exact scaling
//          by 4 commutes with the rounding) and 4 th below (tanh(th) rounds to th in
//          fp32 there). Both forms are checked against torch for every fp16 input.
// The project_fused contract (SRC == KSD_F32) is the reference's Triton kernel as compiled
// for gfx950, which contracts multiply/add pairs: there the Horner steps are fused
// multiply-adds (fp32 in 'fp32', fp16 in 'fp16') and x + (poly + warped) ps is one fp32
// fused multiply-add (rounded to fp16 after it in 'fp16').
// A block is 4 waves; a wave walks RT consecutive rows, a lane owns 8 consecutive charts
// (its per-chart constants stay in registers), a group is G/8 adjacent lanes.
template <int MODE>
__device__ __forceinline__ float tanh_fwd(float v, const uint16_t *tab, bool times4) {
  if constexpr (MODE == 0) {
    return times4 ? 4.0f * tanhf(v) : tanhf(v);
  } else {
    const uint32_t u = f16_bits(v), m = u & 0x7fffu;
    if (m > 0x7c00u) return v;                                      // NaN
    if (times4 && m < 0x0c00u) return 4.0f * v;                     // |th| < 2^-12
    const float t = f16_to_f32(tab[min(m, (uint32_t)KSD_TANH16_LIMIT)]);
    const float r = times4 ? 4.0f * t : t;
    return (u & 0x8000u) ? -r : r;
  }
}

template <int MODE, int SRC, int G, bool VEC, int RT>
__global__ __launch_bounds__(256) void ks3_spine_float_kernel(
    const void *__restrict__ xin, int M, int Fn, const int8_t *__restrict__ codes,
    const uint16_t *__restrict__ ps16, const float *__restrict__ scv, const float *__restrict__ shv,
    float *__restrict__ h_out, int8_t *__restrict__ hq, uint16_t *__restrict__ hs, int ngroups) {
  constexpr int LPG = G / 8;
  __shared__ uint16_t tab[MODE == 1 ? KSD_TANH16_LIMIT + 2 : 2];
  if constexpr (MODE == 1) {
    for (int i = threadIdx.x; i <= KSD_TANH16_LIMIT; i += 256) tab[i] = kTanh16[i];
    __syncthreads();
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = ((int)blockIdx.x * 4 + wave) * RT;
  if (row0 >= M) return;  // wave-uniform, after the block's only barrier
  const int k0 = ((int)blockIdx.y * 64 + (int)(threadIdx.x & 63)) * 8;
  // per-chart constants of the lane's 8 charts (0 past F)
  float A[8], B[8], C0[8], C2[8], C4[8], C5[8], PS[8], SC[8], SH[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int f = k0 + e;
    const bool ok = f < Fn;
    const int fc = ok ? f : 0;
    const float c0 = codes[6 * fc], c1 = codes[6 * fc + 1], c2 = codes[6 * fc + 2];
    const float c3 = codes[6 * fc + 3], c4 = codes[6 * fc + 4], c5 = codes[6 * fc + 5];
    // the combinations are small integers, exact in fp32 and in fp16 (|a| <= 762)
    A[e] = ok ? 2.0f * c0 - 2.0f * c1 + c2 + c3 : 0.0f;
    B[e] = ok ? -3.0f * c0 + 3.0f * c1 - 2.0f * c2 - c3 : 0.0f;
    C0[e] = ok ? c0 : 0.0f;
    C2[e] = ok ? c2 : 0.0f;
    C4[e] = ok ? c4 : 0.0f;
    C5[e] = ok ? c5 : 0.0f;
    PS[e] = ok ? f16_to_f32(ps16[fc]) : 0.0f;
    SC[e] = ok ? scv[fc] : 0.0f;
    SH[e] = ok ? shv[fc] : 0.0f;
  }
#pragma unroll 1
  for (int i = 0; i < RT; ++i) {
    const int row = row0 + i;
    if (row >= M) break;  // wave-uniform
    float x[8], hv[8];
    if constexpr (SRC == KSD_F16) {
      const uint16_t *xr = (const uint16_t *)xin + (int64_t)row * Fn;
      if (VEC && k0 < Fn) {
        const uint4 w = *(const uint4 *)(xr + k0);
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = f16_to_f32((uint16_t)(ww[e / 2] >> (16 * (e & 1))));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = k0 + e < Fn ? f16_to_f32(xr[k0 + e]) : 0.0f;
      }
    } else {
      const float *xr = (const float *)xin + (int64_t)row * Fn;
      if (VEC && k0 < Fn) {
        const float4 a = *(const float4 *)(xr + k0), b = *(const float4 *)(xr + k0 + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = k0 + e < Fn ? xr[k0 + e] : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = fminf(fmaxf(x[e], -kScaleMax), kScaleMax);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v;
      if constexpr (MODE == 0 && SRC == KSD_F32) {
        // ks3_triton.py:91-96 as compiled for gfx950: every Horner step and the final
        // x + s * ps are fused multiply-adds
        const float t = tanh_fwd<0>(x[e] * 0.25f, tab, true);
        const float z = tanh_fwd<0>(SC[e] * (t + SH[e]), tab, false);
        const float poly = fmaf(fmaf(fmaf(A[e], t, B[e]), t, C2[e]), t, C0[e]);
        float wp = fmaf(4.0f * C5[e], z, 2.0f * C4[e]);
        wp = fmaf(wp, z, -(3.0f * C5[e]));
        wp = fmaf(wp, z, -C4[e]);
        v = fmaf(poly + wp, PS[e], x[e]);
        v = v < 0.0f ? 0.0f : v;
        v = v * v;
      } else if constexpr (MODE == 0) {
        const float t = tanh_fwd<0>(x[e] * 0.25f, tab, true);
        const float z = tanh_fwd<0>(SC[e] * (t + SH[e]), tab, false);
        float poly = A[e] * t + B[e];
        poly = poly * t + C2[e];
        poly = poly * t + C0[e];
        float wp = 4.0f * C5[e] * z + 2.0f * C4[e];
        wp = wp * z - 3.0f * C5[e];
        wp = wp * z - C4[e];
        v = x[e] + (poly + wp) * PS[e];
        v = v < 0.0f ? 0.0f : v;
        v = v * v;
      } else if constexpr (SRC == KSD_F32) {
        // ks3_triton.py:77-89 as compiled for gfx950: the six Horner steps are fp16 fused
        // multiply-adds (v_pk_fma_f16) and x + s * ps one fp32 fused multiply-add, rounded
        // to fp16 after it
        typedef _Float16 f16t;
        const float th = f16_round(x[e] * 0.25f);
        const float t = f16_round(tanh_fwd<1>(th, tab, true));
        const float warp = f16_round(SC[e] * (t + SH[e]));
        const float z = tanh_fwd<1>(warp, tab, false);
        const f16t t16 = (f16t)t, z16 = (f16t)z;
        f16t poly = __builtin_fmaf16((f16t)A[e], t16, (f16t)B[e]);
        poly = __builtin_fmaf16(poly, t16, (f16t)C2[e]);
        poly = __builtin_fmaf16(poly, t16, (f16t)C0[e]);
        f16t wp = __builtin_fmaf16((f16t)(4.0f * C5[e]), z16, (f16t)(2.0f * C4[e]));
        wp = __builtin_fmaf16(wp, z16, (f16t)(-3.0f * C5[e]));
        wp = __builtin_fmaf16(wp, z16, (f16t)(-C4[e]));
        v = f16_round(fmaf((float)poly + (float)wp, PS[e], x[e]));
        v = v < 0.0f ? 0.0f : v;
        v = f16_round(v * v);
      } else {
        const float th = f16_round(x[e] * 0.25f);
        const float t = f16_round(tanh_fwd<1>(th, tab, true));
        const float warp = f16_round(SC[e] * (t + SH[e]));
        const float z = tanh_fwd<1>(warp, tab, false);
        float poly = f16_round(f16_round(A[e] * t) + B[e]);
        poly = f16_round(f16_round(poly * t) + C2[e]);
        poly = f16_round(f16_round(poly * t) + C0[e]);
        float wp = f16_round(f16_round(4.0f * C5[e] * z) + 2.0f * C4[e]);
        wp = f16_round(f16_round(wp * z) - 3.0f * C5[e]);
        wp = f16_round(f16_round(wp * z) - C4[e]);
        v = f16_round(x[e] + (poly + wp) * PS[e]);
        v = v < 0.0f ? 0.0f : v;
        v = f16_round(v * v);
      }
      hv[e] = k0 + e < Fn ? v : 0.0f;
    }
    if (h_out) {
      float *hr = h_out + (int64_t)row * Fn;
      if (VEC && k0 < Fn) {
        *(float4 *)(hr + k0) = make_float4(hv[0], hv[1], hv[2], hv[3]);
        *(float4 *)(hr + k0 + 4) = make_float4(hv[4], hv[5], hv[6], hv[7]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (k0 + e < Fn) hr[k0 + e] = hv[e];
      }
    }
    if (hq) {  // quantize_last_dim(h): the group's lanes share one amax (all lanes active)
      const uint32_t am = group_max_u32<LPG>(__builtin_bit_cast(uint32_t, abs_max<8>(hv)));
      const float s = group_scale(__builtin_bit_cast(float, am));
      if (VEC) {
        uint32_t qw[2];
        codes_rcp_packed<8>(hv, s, qw);
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        u32x2 q;
        q.x = qw[0];
        q.y = qw[1];
        __builtin_amdgcn_raw_buffer_store_b64(q, rsrc(hq + (int64_t)row * Fn, Fn),
                                              k0 < Fn ? (uint32_t)k0 : kOob, 0, 0);
      } else if (k0 < Fn) {
        int8_t q[8];
        codes_rcp<8>(hv, s, q);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (k0 + e < Fn) hq[(int64_t)row * Fn + k0 + e] = q[e];
      }
      if (k0 < Fn && (k0 / 8) % LPG == 0) hs[(int64_t)row * ngroups + k0 / G] = scale_bits(s);
    }
  }
}

template <int MODE, int SRC, int G>
static void launch_spine_float(bool vec, dim3 grid, hipStream_t st, const void *x, int64_t M,
                               int64_t F, const int8_t *codes, const uint16_t *ps,
                               const float *sc, const float *sh, float *h, int8_t *hq,
                               uint16_t *hs, int64_t ng) {
  constexpr int RT = 16;
  if (vec)
    hipLaunchKernelGGL((ks3_spine_float_kernel<MODE, SRC, G, true, RT>), grid, dim3(256), 0, st, x,
                       (int)M, (int)F, codes, ps, sc, sh, h, hq, hs, (int)ng);
  else
    hipLaunchKernelGGL((ks3_spine_float_kernel<MODE, SRC, G, false, RT>), grid, dim3(256), 0, st, x,
                       (int)M, (int)F, codes, ps, sc, sh, h, hq, hs, (int)ng);
}
constexpr int kSpineFloatRows = 4 * 16;  // rows per block of ks3_spine_float_kernel

// ---------------------------------------------------------------- gradient handoff
// _grad_handoff (ks3_int8.py:75-84) without a host round trip: the fp16 conversion of a
// gradient is used when every element of it is finite, else the fp32 gradient itself. The
// decision is one device flag (set by any element whose fp16 conversion overflows or is
// NaN; the caller zeroes it), read by the selecting pass; the result is written as fp32,
// the masters' dtype, which is what autograd makes of either branch.
__global__ __launch_bounds__(256) void handoff_flag_kernel(const float *__restrict__ t, int64_t n,
                                                           int *__restrict__ flag) {
  bool bad = false;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const uint16_t h = f16_bits(t[i]);
    bad |= (h & 0x7c00u) == 0x7c00u;  // inf or NaN in fp16
  }
  if (__syncthreads_or(bad) && threadIdx.x == 0) atomicOr(flag, 1);
}

__global__ __launch_bounds__(256) void handoff_select_kernel(const float *__restrict__ t, int64_t n,
                                                             const int *__restrict__ flag,
                                                             float *__restrict__ out) {
  const bool keep32 = *flag != 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float v = t[i];
    out[i] = keep32 ? v : f16_round(v);
  }
}

// out != t: one pass writes fp16(t) and raises the flag; the fix-up pass then rewrites t
// when the flag is set (every block returns at once when it is not). One read of t fewer
// than the flag + select passes.
__global__ __launch_bounds__(256) void handoff_round_kernel(const float *__restrict__ t, int64_t n,
                                                            int *__restrict__ flag, float *__restrict__ out) {
  bool bad = false;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float v = t[i];
    bad |= (f16_bits(v) & 0x7c00u) == 0x7c00u;  // inf or NaN in fp16
    out[i] = f16_round(v);
  }
  if (__syncthreads_or(bad) && threadIdx.x == 0) atomicOr(flag, 1);
}

__global__ __launch_bounds__(256) void handoff_fixup_kernel(const float *__restrict__ t, int64_t n,
                                                            const int *__restrict__ flag,
                                                            float *__restrict__ out) {
  if (*flag == 0) return;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) out[i] = t[i];
}

}  // namespace ksd

using namespace ksd;

// The fused contract's per-chart increment table (F x 256 fp32), for the fused projection
// GEMM in gemm.hip.
int ksd::ks3_fused_table(const int8_t *spine_codes, const uint16_t *spine_scale,
                         const uint16_t *warp_scale, const uint16_t *warp_shift, const int8_t *tanh_lut,
                         int64_t F, float *table, hipStream_t st) {
  hipLaunchKernelGGL(ks3_spine_table_kernel<true>, dim3((unsigned)F), dim3(256), 0, st, spine_codes,
                     spine_scale, warp_scale, warp_shift, tanh_lut, (void *)table);
  return check_launch("ks3_project_fused (table)");
}

static int spine_checks(const char *who, const void *in, int64_t M, int64_t F, const int8_t *spine_codes,
                        const uint16_t *spine_scale, const uint16_t *warp_scale,
                        const uint16_t *warp_shift, const int8_t *tanh_lut, int group,
                        const void *table) {
  if (M < 0 || F < 0) return fail(KSD_EINVAL, "%s: negative shape (%lld, %lld)", who, (long long)M, (long long)F);
  if (!valid_group(group)) return fail(KSD_EINVAL, "%s: group must be 32, 64 or 128", who);
  if (!in || !spine_codes || !spine_scale || !warp_scale || !warp_shift || !tanh_lut)
    return fail(KSD_EINVAL, "%s: null input pointer", who);
  if (!table || ((uintptr_t)table & 15) != 0)
    return fail(KSD_EINVAL, "%s: table workspace must be a 16-byte aligned buffer", who);
  // stores address a block's kSpineRows rows from one base with 32-bit offsets
  if (F > (1LL << 31) / (2 * kSpineRows)) return fail(KSD_EINVAL, "%s: F too large", who);
  if (((uintptr_t)tanh_lut & 3) != 0) return fail(KSD_EINVAL, "%s: tanh_lut must be 4-byte aligned", who);
  if (cdiv(M, kSpineRows) > 0x7fffffff) return fail(KSD_EINVAL, "%s: M too large", who);
  return KSD_OK;
}

extern "C" int ksd_ks3_spine_fwd(const uint16_t *coords, int64_t M, int64_t F,
                                 const int8_t *spine_codes, const uint16_t *spine_scale,
                                 const uint16_t *warp_scale, const uint16_t *warp_shift,
                                 const int8_t *tanh_lut, int group, float *h, int8_t *h_codes,
                                 uint16_t *h_scales, uint16_t *table, void *stream) {
  int rc = spine_checks("ks3_spine_fwd", coords, M, F, spine_codes, spine_scale, warp_scale,
                        warp_shift, tanh_lut, group, table);
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
  hipLaunchKernelGGL(ks3_spine_table_kernel<false>, dim3((unsigned)F), dim3(256), 0, st, spine_codes,
                     spine_scale, warp_scale, warp_shift, tanh_lut, (void *)table);
#define KSD_SPINE_ARGS vec, grid, st, coords, M, F, table, h, h_codes, h_scales, ng
  switch (group) {
    case 32: launch_spine<32>(KSD_SPINE_ARGS); break;
    case 64: launch_spine<64>(KSD_SPINE_ARGS); break;
    default: launch_spine<128>(KSD_SPINE_ARGS); break;
  }
#undef KSD_SPINE_ARGS
  return check_launch("ks3_spine_fwd");
}

// ---------------------------------------------------------------- no-allocation variant
// ksd_ks3_spine_fwd_noalloc runs ksd_ks3_spine_fwd with its per-chart increment table in
// `scratch`, a file-scope device array of kScratchCharts x 256 fp16 (4 MiB), of which every
// GPU the library runs on holds its own copy until the process ends. The table kernel of
// each call rewrites every entry the element pass reads (rows below F), so nothing needs
// clearing; calls that overlap on one GPU share the array and race. Host code never passes
// the array's name to a kernel: its device address comes from hipGetSymbolAddress, once
// per device, with that device current.
constexpr int64_t kScratchCharts = 8192;
static __device__ __align__(256) uint16_t scratch[kScratchCharts * 256];
static uint16_t *g_scratch_addr[64];  // per device ordinal

static int scratch_table(const char *who, hipStream_t st, uint16_t **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(KSD_EHIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(KSD_EINVAL, "%s: device ordinal %d out of range", who, dev);
  if (st != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return fail(KSD_EHIP, "%s: hipStreamGetDevice: %s", who, hipGetErrorString(e));
    if (sdev != dev)
      return fail(KSD_EINVAL, "%s: the stream belongs to device %d but device %d is current", who,
                  sdev, dev);
  }
  uint16_t *p = __atomic_load_n(&g_scratch_addr[dev], __ATOMIC_ACQUIRE);
  if (p == nullptr) {
    void *q = nullptr;
    e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
    if (e != hipSuccess || q == nullptr)
      return fail(KSD_EHIP, "%s: hipGetSymbolAddress(scratch): %s", who, hipGetErrorString(e));
    p = (uint16_t *)q;
    __atomic_store_n(&g_scratch_addr[dev], p, __ATOMIC_RELEASE);
  }
  *out = p;
  return KSD_OK;
}

extern "C" int ksd_ks3_spine_fwd_noalloc(const uint16_t *coords, int64_t M, int64_t F,
                                         const int8_t *spine_codes, const uint16_t *spine_scale,
                                         const uint16_t *warp_scale, const uint16_t *warp_shift,
                                         const int8_t *tanh_lut, int group, float *h,
                                         int8_t *h_codes, uint16_t *h_scales, void *stream) {
  if (F > kScratchCharts)
    return fail(KSD_EINVAL, "ks3_spine_fwd_noalloc: F=%lld charts exceeds the %lld-chart scratch table",
                (long long)F, (long long)kScratchCharts);
  if (F < 0 || M < 0)
    return fail(KSD_EINVAL, "ks3_spine_fwd_noalloc: negative shape (%lld, %lld)", (long long)M, (long long)F);
  uint16_t *table = nullptr;
  const int rc = scratch_table("ks3_spine_fwd_noalloc", (hipStream_t)stream, &table);
  if (rc) return rc;
  return ksd_ks3_spine_fwd(coords, M, F, spine_codes, spine_scale, warp_scale, warp_shift, tanh_lut,
                           group, h, h_codes, h_scales, table, stream);
}

extern "C" int ksd_ks3_spine_fused(const float *acc, int64_t M, int64_t F,
                                   const int8_t *spine_codes, const uint16_t *spine_scale,
                                   const uint16_t *warp_scale, const uint16_t *warp_shift,
                                   const int8_t *tanh_lut, int group, int8_t *h_codes,
                                   uint16_t *h_scales, float *table, void *stream) {
  int rc = spine_checks("ks3_spine_fused", acc, M, F, spine_codes, spine_scale, warp_scale,
                        warp_shift, tanh_lut, group, table);
  if (rc) return rc;
  if (!h_codes || !h_scales) return fail(KSD_EINVAL, "ks3_spine_fused: null output pointer");
  if (M == 0 || F == 0) return KSD_OK;
  const bool vec = (F & 3) == 0 && ((uintptr_t)acc & 15) == 0 && ((uintptr_t)h_codes & 3) == 0;
  const int64_t ng = cdiv(F, group);
  dim3 grid((unsigned)cdiv(F, 128), (unsigned)cdiv(M, kSpineRows));
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(ks3_spine_table_kernel<true>, dim3((unsigned)F), dim3(256), 0, st, spine_codes,
                     spine_scale, warp_scale, warp_shift, tanh_lut, (void *)table);
#define KSD_FUSED_ARGS vec, grid, st, acc, M, F, table, h_codes, h_scales, ng
  switch (group) {
    case 32: launch_fused<32>(KSD_FUSED_ARGS); break;
    case 64: launch_fused<64>(KSD_FUSED_ARGS); break;
    default: launch_fused<128>(KSD_FUSED_ARGS); break;
  }
#undef KSD_FUSED_ARGS
  return check_launch("ks3_spine_fused");
}

extern "C" int ksd_ks3_spine_float(const void *x, int x_dtype, int64_t M, int64_t F,
                                   const int8_t *spine_codes, const uint16_t *spine_scale,
                                   const float *warp_scale, const float *warp_shift, int mode,
                                   int group, float *h, int8_t *h_codes, uint16_t *h_scales,
                                   void *stream) {
  if (M < 0 || F < 0) return fail(KSD_EINVAL, "ks3_spine_float: negative shape");
  if (!valid_group(group)) return fail(KSD_EINVAL, "ks3_spine_float: group must be 32, 64 or 128");
  if (mode != 0 && mode != 1) return fail(KSD_EINVAL, "ks3_spine_float: mode must be 0 (fp32) or 1 (fp16)");
  if (x_dtype != KSD_F16 && x_dtype != KSD_F32)
    return fail(KSD_ETYPE, "ks3_spine_float: x must be fp16 coordinates or the fp32 accumulator");
  if (!x || !spine_codes || !spine_scale || !warp_scale || !warp_shift)
    return fail(KSD_EINVAL, "ks3_spine_float: null input pointer");
  if ((h_codes == nullptr) != (h_scales == nullptr))
    return fail(KSD_EINVAL, "ks3_spine_float: h_codes and h_scales go together");
  if (!h && !h_codes) return fail(KSD_EINVAL, "ks3_spine_float: no output requested");
  if (M == 0 || F == 0) return KSD_OK;
  if (F > (1LL << 28) || M > 0x7fffffffLL - kSpineFloatRows)
    return fail(KSD_EINVAL, "ks3_spine_float: too large");
  const size_t esz = x_dtype == KSD_F32 ? 4 : 2;
  const bool vec = (F & 7) == 0 && ((uintptr_t)x % 16) == 0 && (F * esz) % 16 == 0 &&
                   ((uintptr_t)h % 16) == 0 && ((uintptr_t)h_codes % 8) == 0;
  const int64_t ng = cdiv(F, group);
  dim3 grid((unsigned)cdiv(M, kSpineFloatRows), (unsigned)cdiv(F, 512));
  hipStream_t st = (hipStream_t)stream;
#define KSD_SFA vec, grid, st, x, M, F, spine_codes, spine_scale, warp_scale, warp_shift, h, h_codes, h_scales, ng
#define KSD_SF_G(MO, SR)                                                  \
  switch (group) {                                                        \
    case 32: launch_spine_float<MO, SR, 32>(KSD_SFA); break;              \
    case 64: launch_spine_float<MO, SR, 64>(KSD_SFA); break;              \
    default: launch_spine_float<MO, SR, 128>(KSD_SFA); break;             \
  }
  if (mode == 0) {
    if (x_dtype == KSD_F16) { KSD_SF_G(0, KSD_F16) } else { KSD_SF_G(0, KSD_F32) }
  } else {
    if (x_dtype == KSD_F16) { KSD_SF_G(1, KSD_F16) } else { KSD_SF_G(1, KSD_F32) }
  }
#undef KSD_SF_G
#undef KSD_SFA
  return check_launch("ks3_spine_float");
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
  hipLaunchKernelGGL(ks3_vjp_finalize_kernel, dim3((unsigned)cdiv(F, 256), 8), dim3(256), 0,
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

extern "C" int ksd_grad_handoff(const float *t, int64_t n, int *flag, float *out, void *stream) {
  if (n < 0) return fail(KSD_EINVAL, "grad_handoff: negative size");
  if (n == 0) return KSD_OK;
  if (!t || !flag || !out) return fail(KSD_EINVAL, "grad_handoff: null pointer");
  const int64_t blocks = cdiv(n, 256 * 8);
  const unsigned grid = (unsigned)(blocks < 4096 ? blocks : 4096);
  hipStream_t st = (hipStream_t)stream;
  if (out != t) {
    hipLaunchKernelGGL(handoff_round_kernel, dim3(grid), dim3(256), 0, st, t, n, flag, out);
    hipLaunchKernelGGL(handoff_fixup_kernel, dim3(grid), dim3(256), 0, st, t, n, (const int *)flag, out);
  } else {  // in place: decide first, then round
    hipLaunchKernelGGL(handoff_flag_kernel, dim3(grid), dim3(256), 0, st, t, n, flag);
    hipLaunchKernelGGL(handoff_select_kernel, dim3(grid), dim3(256), 0, st, t, n, (const int *)flag, out);
  }
  return check_launch("grad_handoff");
}
