// GS symmetric int8 quantization kernels for gfx950.
//
// Contract (reference ksdraft/kernels/quant.py:30-52): per row, per `group`-wide slice
// of the last dim, amax -> scale = fp16(clamp(amax/127, 2^-24, 65504)) -> code =
// clamp(rne(x/scale), -127, 127). A partial last group is zero-padded for the amax and
// its padded lanes are not stored. These kernels are HBM-streaming: coalesced 16-byte
// loads, wave shuffles for the group amax, no LDS for the row-wise form.
#include "ksd_common.h"

namespace ksd {

// ----------------------------------------------------------------------------------
// Row-wise quantization: one group is owned by G/8 consecutive lanes, 8 elements each.
template <int DT, int G, bool VEC>
__global__ __launch_bounds__(256) void quant_rows_kernel(
    const void *__restrict__ xv, int64_t rows, int64_t K, int64_t stride, int64_t ngroups,
    int8_t *__restrict__ codes, uint16_t *__restrict__ scales,
    const float *__restrict__ noise, float dither2) {
  using T = typename Elem<DT>::T;
  constexpr int LPG = G / 8;
  const T *x = (const T *)xv;
  const int64_t gid = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPG;
  const int sub = threadIdx.x % LPG;
  const bool active = gid < rows * ngroups;
  const int64_t row = active ? gid / ngroups : 0;
  const int64_t grp = active ? gid % ngroups : 0;
  const int64_t k0 = grp * G + sub * 8;
  const T *xr = x + row * stride;

  float v[8];
  const bool full = active && (k0 + 8 <= K);
  if (VEC && full) {
    if constexpr (sizeof(T) == 4) {
      const float4 *p = (const float4 *)(xr + k0);
      float4 a = p[0], b = p[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      uint4 a = *(const uint4 *)(xr + k0);
      const uint16_t *h = (const uint16_t *)&a;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = Elem<DT>::load(h + i);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = (active && k0 + i < K) ? Elem<DT>::load(xr + k0 + i) : 0.0f;
  }

  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = amax2(amax, fabsf(v[i]));
#pragma unroll
  for (int off = LPG / 2; off > 0; off >>= 1) amax = amax2(amax, __shfl_xor(amax, off));
  const float s = group_scale(amax);

  int8_t q[8];
  if (noise != nullptr) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // stages.py:44-47: codes + (rand - 0.5) * (2*dither), fp32 ops, separately rounded
      float c = v[i] / s;
      if (active) c = c + (noise[row * ngroups * G + k0 + i] - 0.5f) * dither2;
      q[i] = code_of(c);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = code_of(v[i] / s);
  }
  if (!active) return;
  int8_t *cr = codes + row * K;
  if (VEC && full) {
    *(uint2 *)(cr + k0) = *(const uint2 *)q;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < K) cr[k0 + i] = q[i];
  }
  if (sub == 0) scales[row * ngroups + grp] = scale_bits(s);
}

// Row-wise quantization, aligned rows without dither: block = 4 waves; a wave walks RT
// consecutive rows, a lane owns 8 consecutive elements (grid.y walks a row in 512-element
// slices, so a group is G/8 adjacent lanes of one wave). The next row is loaded from a
// clamped valid address while the current one is encoded; stores go through buffer
// resources, lanes past K (or not leading their group, for the scale) getting an offset
// past num_records, so no store sits in a branch and no wait covers the stores.
// Requires K % 8 == 0, 16-byte aligned rows and 8-byte aligned code rows.
template <int DT, int G, int RT>
__global__ __launch_bounds__(256) void quant_rows_fast_kernel(
    const void *__restrict__ xv, int64_t rows, int K, int64_t stride, int ngroups,
    int8_t *__restrict__ codes, uint16_t *__restrict__ scales) {
  using T = typename Elem<DT>::T;
  constexpr int LPG = G / 8;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * RT;
  if (row0 >= rows) return;                                   // wave-uniform
  const int k0 = ((int)blockIdx.y * 64 + (int)(threadIdx.x & 63)) * 8;
  const bool kok = k0 < K;
  const T *xb = (const T *)xv + (kok ? k0 : 0);
  const bool lead = kok && (k0 / 8) % LPG == 0;
  Raw8<DT> rn = load_raw8<DT>(xb + row0 * stride);
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int64_t row = row0 + i;
    if (row >= rows) break;                                   // wave-uniform
    float v[8];
    cvt_raw8<DT>(rn, kok, v);
    if (i + 1 < RT) rn = load_raw8<DT>(xb + min(row + 1, rows - 1) * stride);
    const uint32_t am = __builtin_bit_cast(uint32_t, abs_max<8>(v));
    const float s = group_scale(__builtin_bit_cast(float, group_max_u32<LPG>(am)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    uint32_t qw[2];
    codes_rcp_packed<8>(v, s, qw);
    u32x2 q;
    q.x = qw[0];
    q.y = qw[1];
    __builtin_amdgcn_raw_buffer_store_b64(q, rsrc(codes + row * K, K), kok ? (uint32_t)k0 : kOob, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rsrc(scales + row * ngroups, 2 * (int64_t)ngroups),
                                          lead ? (uint32_t)(k0 / G) * 2 : kOob, 0, 0);
  }
}

// ----------------------------------------------------------------------------------
// Dequantization: out = float(code) * float(scale), exact in fp32 (quant.py:66).
__global__ __launch_bounds__(256) void dequant_rows_kernel(
    const int8_t *__restrict__ codes, const uint16_t *__restrict__ scales, int64_t rows,
    int64_t K, int64_t nsc, int group, float *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * K) return;
  const int64_t r = i / K, k = i % K;
  const int64_t g = k / group;
  const float s = g < nsc ? f16_to_f32(scales[r * nsc + g]) : 0.0f;
  out[i] = (float)codes[i] * s;
}

// ----------------------------------------------------------------------------------
// Transposed quantization: codes (C, R) = quantize along R of x (R, C); with an int8 source
// the values are dequantized first (requant: float(code) * float(scale), exact).
//
// A 256-thread block owns one G-row group by 64 columns. Loads are 16 bytes per lane along
// C (a wave covers whole 64-column row segments); the tile goes to LDS transposed (a skewed
// column layout keeps writes and reads free of bank conflicts); then 4 lanes per column
// reduce the group amax with two shuffles and each stores G/4 contiguous codes, so an
// output row receives G contiguous bytes from 4 adjacent lanes.
enum { SRC_F32 = 0, SRC_BF16 = 1, SRC_F16 = 2, SRC_I8 = 3 };

template <int SRC, int G>
__device__ __forceinline__ void quant_T_tile(
    const void *__restrict__ xv, const uint16_t *__restrict__ in_scales, int64_t nsc_in,
    int gin, int64_t R, int64_t C, int64_t nbc, int64_t ngr, int8_t *__restrict__ codes,
    uint16_t *__restrict__ scales, bool rows_vec, int64_t bid) {
  // LDS column layout: column c at c * PITCH, row r at + r + SKEW(r). For G = 128 the
  // pitch is 145 (17 mod 64 banks) and rows >= 64 are shifted by 16: the transposing
  // writes (a wave covers 4..16 rows of 16..4 column quads) and the group reads (lanes =
  // 16 columns x 4 quarter-groups of 32 rows) both hit 64 distinct banks. For G <= 64 the
  // pitch is G + 1 with no shift (the quarter-groups are then 16 rows or fewer apart).
  constexpr int PITCH = G == 128 ? 145 : G + 1;
  __shared__ float tile[64 * PITCH];
  auto lds_at = [](int c, int r) { return c * PITCH + r + (G == 128 && r >= 64 ? 16 : 0); };
  const int tid = threadIdx.x;
  const int64_t bc = bid % nbc, br = bid / nbc;
  const int64_t r0 = br * G, c0 = bc * 64;

  // ---- load: EPV elements per 16-byte vector, LPR lanes per 64-column row segment
  constexpr int EPV = SRC == SRC_F32 ? 4 : SRC == SRC_I8 ? 16 : 8;
  constexpr int LPR = 64 / EPV, RPP = 256 / LPR;  // rows per pass
  const int tx = tid % LPR, ty = tid / LPR;
  const int64_t cb = c0 + tx * EPV;  // first column of this lane's vector
  constexpr int NP = G >= RPP ? G / RPP : 1;  // passes (with RPP > G, rows ty >= G idle)
  const bool ty_ok = ty < G;
  float v[NP][EPV];
  if (rows_vec && r0 + G <= R && c0 + 64 <= C && ty_ok) {
    // interior tile: every load a 16-byte vector, all issued before any LDS write
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      const int64_t gr = r0 + ty + pass * RPP;
      if constexpr (SRC == SRC_F32) {
        const float4 a = *(const float4 *)((const float *)xv + gr * C + cb);
        v[pass][0] = a.x; v[pass][1] = a.y; v[pass][2] = a.z; v[pass][3] = a.w;
      } else if constexpr (SRC == SRC_I8) {
        const int4 a = *(const int4 *)((const int8_t *)xv + gr * C + cb);
        const float sc = f16_to_f32(in_scales[gr * nsc_in + cb / gin]);
        const int w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) v[pass][i] = (float)(int8_t)(w[i >> 2] >> ((i & 3) * 8)) * sc;
      } else {
        const uint4 a = *(const uint4 *)((const uint16_t *)xv + gr * C + cb);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint16_t h = (uint16_t)(w[i >> 1] >> ((i & 1) * 16));
          v[pass][i] = SRC == SRC_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
      }
    }
  } else {
    // ragged or unaligned tile: element loads, zeros outside the tensor
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      const int64_t gr = r0 + ty + pass * RPP;
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const int64_t gc = cb + i;
        float x = 0.0f;
        if (ty_ok && gr < R && gc < C) {
          if constexpr (SRC == SRC_F32) x = ((const float *)xv)[gr * C + gc];
          else if constexpr (SRC == SRC_BF16) x = bf16_to_f32(((const uint16_t *)xv)[gr * C + gc]);
          else if constexpr (SRC == SRC_F16) x = f16_to_f32(((const uint16_t *)xv)[gr * C + gc]);
          else x = (float)((const int8_t *)xv)[gr * C + gc] * f16_to_f32(in_scales[gr * nsc_in + gc / gin]);
        }
        v[pass][i] = x;
      }
    }
  }
  if (ty_ok) {
#pragma unroll
    for (int pass = 0; pass < NP; ++pass)
#pragma unroll
      for (int i = 0; i < EPV; ++i) tile[lds_at(tx * EPV + i, ty + pass * RPP)] = v[pass][i];
  }
  __syncthreads();

  // ---- column c = tid / 4, rows [part * G/4, +G/4)
  constexpr int RPT = G / 4;
  const int c = tid >> 2, part = tid & 3;
  float col[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) col[j] = tile[lds_at(c, part * RPT + j)];
  const uint32_t am = __builtin_bit_cast(uint32_t, abs_max<RPT>(col));
  const float s = group_scale(__builtin_bit_cast(float, group_max_u32<4>(am)));
  const int64_t gc = c0 + c;
  if (gc >= C) return;
  if (part == 0) scales[gc * ngr + br] = scale_bits(s);
  uint32_t w[RPT / 4];
  codes_rcp_packed<RPT>(col, s, w);
  int8_t *dst = codes + gc * R + r0 + part * RPT;
  const int64_t rbase = r0 + part * RPT;
  if (rbase + RPT <= R && (((uintptr_t)dst) % (RPT < 16 ? RPT : 16)) == 0) {
    if constexpr (RPT == 8) {
      *(uint2 *)dst = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
      for (int j = 0; j < RPT / 4; j += 4) *(uint4 *)(dst + 4 * j) = make_uint4(w[j], w[j + 1], w[j + 2], w[j + 3]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < RPT; ++j)
      if (rbase + j < R) dst[j] = (int8_t)(w[j / 4] >> (8 * (j % 4)));
  }
}

template <int SRC, int G>
__global__ __launch_bounds__(256) void quant_T_kernel(
    const void *__restrict__ xv, const uint16_t *__restrict__ in_scales, int64_t nsc_in,
    int gin, int64_t R, int64_t C, int64_t nbc, int64_t ngr, int8_t *__restrict__ codes,
    uint16_t *__restrict__ scales, bool rows_vec) {
  quant_T_tile<SRC, G>(xv, in_scales, nsc_in, gin, R, C, nbc, ngr, codes, scales, rows_vec, blockIdx.x);
}

// requant_transpose (group 128 in and out) of many int8 tensors in one launch: the weight
// transposes a training step's backward needs, built once per optimizer step. A batch
// travels by value in the kernel arguments; a block finds its tensor with scalar compares.
constexpr int kRqtBatch = 32;
struct RqtArg {
  const int8_t *x;
  const uint16_t *s;
  int8_t *codes;
  uint16_t *scales;
  int64_t R, C, nbc, ngr;
  int32_t first_block, rv;
};
struct RqtBatchArg {
  RqtArg t[kRqtBatch];
  int32_t n;
};
__global__ __launch_bounds__(256) void requant_T_multi_kernel(const RqtBatchArg b) {
  int i = 0;
  for (int k = 1; k < b.n; ++k)
    if (b.t[k].first_block <= (int)blockIdx.x) i = k;
  const RqtArg &t = b.t[i];
  quant_T_tile<SRC_I8, 128>(t.x, t.s, (t.C + 127) / 128, 128, t.R, t.C, t.nbc, t.ngr, t.codes, t.scales,
                            t.rv != 0, (int64_t)blockIdx.x - t.first_block);
}

// ----------------------------------------------------------------------------------
// Dual-layout quantization, G = 128: one pass over a 128 x 128 tile of x (R, C) emits the
// row codes (quantize_last_dim(x), along C) and the column codes (along R) of x itself
// (quantize_last_dim(x.t())); the X^T recipe quant(dequant(quant(X))^T) has its own
// kernel, quant_dual_codes_kernel, below. The rows are
// quantized from registers (16 lanes per row, 8 elements each), the values then go to LDS
// transposed in quant_T_kernel's conflict-free layout, and 4 lanes per column quantize the
// columns. Requires C % 8 == 0 and 16-byte aligned rows; rows past R read as zeros and
// are not stored.
// Cross-entropy backward source of the dual kernel: x[r, c] is not read from memory but
// formed from fp32 logits y and per-row softmax statistics,
//   dY[r, c] = (exp(y[r, c] - max_r) / sum_r - [c == t_r]) * w_r,
// with w_r = grad_scale for a row whose target is in range and not ignore_index, else 0.
struct CeSrc {
  const float *rmax, *rinv;  // max_r and 1 / sum_r (ce_row_stats_kernel)
  const int64_t *tgt;
  int64_t ignore;
  const float *gscale;       // device scalar: d loss / d (mean CE), divided by the row count
  float *dy;                 // optional fp32 copy of dY (R, C), nullptr when not wanted
};
constexpr float kLog2e = 1.4426950408889634f;

// col_part (optional, not with CE): (ceil(R/128), C) fp32 partial column sums of x, one row
// per 128-row tile, each the sum of its four 32-row parts ((p0 + p1) + (p2 + p3)), every
// part summed in row order; colsum_finalize_kernel adds the tiles in order.
// H16: quantize the fp16 rounding of x (x.to(float16) first: the KS3 cell's backward
// quantizes its upstream gradient as g16 = grad.to(float16), ks3_int8.py:345-348, :421-422).
template <int DT, bool CE = false, bool H16 = false>
__global__ __launch_bounds__(512) void quant_dual_kernel(
    const void *__restrict__ xv, int64_t R, int64_t C, int8_t *__restrict__ codes,
    uint16_t *__restrict__ scales, int8_t *__restrict__ codes_t, uint16_t *__restrict__ scales_t,
    CeSrc ce = CeSrc{}, float *__restrict__ col_part = nullptr) {
  using T = typename Elem<DT>::T;
  constexpr int G = 128, PITCH = 145;
  __shared__ float tile[128 * PITCH];
  auto lds_at = [](int c, int r) { return c * PITCH + r + (r >= 64 ? 16 : 0); };
  const int tid = threadIdx.x;
  const int64_t c0 = (int64_t)blockIdx.x * 128, r0 = (int64_t)blockIdx.y * 128;
  const int64_t ngC = (C + G - 1) / G, ngR = (R + G - 1) / G;
  // the tile's rows as wave-uniform buffer descriptors (per-lane offsets below 2^31: the
  // host checks 128 * C * 4): a per-lane base would wrap every store in a readfirstlane loop
  const int64_t nrows = min((int64_t)128, R - r0);
  const auto rq = rsrc(codes + r0 * C, nrows * C);
  const auto rs = rsrc(scales + r0 * ngC, 2 * nrows * ngC);

  // ---- rows: lane (rr, sub) takes rows r0 + 32 p + rr (p = 0..3), columns c0 + 8 sub .. + 8;
  // the four rows' loads are issued before any arithmetic
  const int rr = tid >> 4, sub = tid & 15;
  const int64_t col = c0 + sub * 8;
  const bool cok = col < C;
  const T *xb = (const T *)xv + (cok ? col : 0);
  Raw8<DT> raw[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) raw[p] = load_raw8<DT>(xb + min(r0 + 32 * p + rr, R - 1) * C);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int lr = 32 * p + rr;  // row within the tile
    const int64_t row = r0 + lr;
    const bool ok = cok && row < R;
    float v[8];
    cvt_raw8<DT>(raw[p], ok, v);
    if constexpr (H16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = f16_round(v[i]);
    }
    if constexpr (CE) {
      const int64_t rs = row < R ? row : R - 1;
      const int64_t t = ce.tgt[rs];
      const bool live = ok && t != ce.ignore && t >= 0 && t < C;
      const float m = ce.rmax[rs], inv = ce.rinv[rs], w = live ? *ce.gscale : 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = __builtin_amdgcn_exp2f((v[i] - m) * kLog2e) * inv;
        v[i] = live ? (e - (col + i == t ? 1.0f : 0.0f)) * w : 0.0f;
      }
      if (ce.dy) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const auto dr = rsrc(ce.dy + r0 * C, 4 * nrows * C);
        const uint32_t off = ok ? (uint32_t)(lr * C + col) * 4 : kOob;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]}), dr, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{v[4], v[5], v[6], v[7]}), dr,
                                               ok ? off + 16 : kOob, 0, 0);
      }
    }
    const uint32_t am = group_max_u32<16>(__builtin_bit_cast(uint32_t, abs_max<8>(v)));
    const float s = group_scale(__builtin_bit_cast(float, am));
    uint32_t w[2];
    codes_rcp_packed<8>(v, s, w);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 q;
    q.x = w[0];
    q.y = w[1];
    __builtin_amdgcn_raw_buffer_store_b64(q, rq, ok ? (uint32_t)(lr * C + col) : kOob, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rs,
                                          ok && sub == 0 ? (uint32_t)(lr * ngC + col / G) * 2 : kOob, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) tile[lds_at(sub * 8 + i, lr)] = v[i];
  }
  __syncthreads();

  // ---- columns: lane (c, part) takes column c, rows part * 32 .. + 32
  constexpr int RPT = 32;
  const int c = tid >> 2, part = tid & 3;
  float colv[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) colv[j] = tile[lds_at(c, part * RPT + j)];
  const uint32_t am = group_max_u32<4>(__builtin_bit_cast(uint32_t, abs_max<RPT>(colv)));
  const float s = group_scale(__builtin_bit_cast(float, am));
  const int64_t gc = c0 + c;
  if (!CE && col_part != nullptr) {  // this tile's sum of column gc (rows past R are zeros)
    float ps = colv[0];
#pragma unroll
    for (int j = 1; j < RPT; ++j) ps += colv[j];
    // the four parts of a column sit in one lane quad: pair sums, then the pairs' sum
    // (a + b == b + a, so both lanes of a pair hold the same value)
    ps += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, ps), 0xB1, 0xF, 0xF, false));
    ps += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, ps), 0x4E, 0xF, 0xF, false));
    if (part == 0 && gc < C) col_part[(int64_t)blockIdx.y * C + gc] = ps;
  }
  if (gc >= C) return;
  if (part == 0) scales_t[gc * ngR + blockIdx.y] = scale_bits(s);
  uint32_t w[RPT / 4];
  codes_rcp_packed<RPT>(colv, s, w);
  int8_t *dst = codes_t + gc * R + r0 + part * RPT;
  const int64_t rbase = r0 + part * RPT;
  if (rbase + RPT <= R && (((uintptr_t)dst) & 15) == 0) {
#pragma unroll
    for (int j = 0; j < RPT / 4; j += 4) *(uint4 *)(dst + 4 * j) = make_uint4(w[j], w[j + 1], w[j + 2], w[j + 3]);
  } else {
#pragma unroll
    for (int j = 0; j < RPT; ++j)
      if (rbase + j < R) dst[j] = (int8_t)(w[j / 4] >> (8 * (j % 4)));
  }
}

// colsum[c] = sum over tiles t = 0, 1, ... of col_part[t, c], in tile order.
__global__ __launch_bounds__(256) void colsum_finalize_kernel(const float *__restrict__ col_part, int64_t ntiles,
                                                              int64_t C, float *__restrict__ colsum) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  float acc = 0.0f;
  for (int64_t t0 = 0; t0 < ntiles; t0 += 16) {  // 16 loads in flight, then the adds in order
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = t0 + i < ntiles ? col_part[(t0 + i) * C + c] : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (t0 + i < ntiles) acc = t0 + i == 0 ? v[i] : acc + v[i];
  }
  colsum[c] = acc;
}

// Dual-layout quantization of an X operand (t_from_codes: the recipe quant(dequant(quant(
// X))^T)) with a small LDS tile: as quant_dual_kernel, but the transposed tile holds the
// row codes as int8, column-major with a 132-byte pitch (an odd word stride: at most 2-way
// bank conflicts on the byte writes and the dword reads), and the 128 row scales; 17.4 KB
// instead of 74 KB, so four blocks fit a CU. The column pass dequantizes code * scale
// (exact in fp32, as in quant_dual_kernel) before its amax and codes.
template <int DT>
__device__ __forceinline__ void dual_codes_tile(
    const void *__restrict__ xv, int64_t R, int64_t C, int8_t *__restrict__ codes,
    uint16_t *__restrict__ scales, int8_t *__restrict__ codes_t, uint16_t *__restrict__ scales_t,
    int64_t bx, int64_t by) {
  using T = typename Elem<DT>::T;
  constexpr int G = 128, PB = 132;
  __shared__ __attribute__((aligned(16))) int8_t tq[128 * PB];  // [column][row]
  __shared__ __attribute__((aligned(16))) float srow[128];
  const int tid = threadIdx.x;
  const int64_t c0 = bx * 128, r0 = by * 128;
  const int64_t ngC = (C + G - 1) / G, ngR = (R + G - 1) / G;
  const int64_t nrows = min((int64_t)128, R - r0);
  const auto rq = rsrc(codes + r0 * C, nrows * C);
  const auto rs = rsrc(scales + r0 * ngC, 2 * nrows * ngC);

  // ---- rows, as in quant_dual_kernel
  const int rr = tid >> 4, sub = tid & 15;
  const int64_t col = c0 + sub * 8;
  const bool cok = col < C;
  const T *xb = (const T *)xv + (cok ? col : 0);
  Raw8<DT> raw[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) raw[p] = load_raw8<DT>(xb + min(r0 + 32 * p + rr, R - 1) * C);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int lr = 32 * p + rr;
    const int64_t row = r0 + lr;
    const bool ok = cok && row < R;
    float v[8];
    cvt_raw8<DT>(raw[p], ok, v);
    const uint32_t am = group_max_u32<16>(__builtin_bit_cast(uint32_t, abs_max<8>(v)));
    const float s = group_scale(__builtin_bit_cast(float, am));
    uint32_t w[2];
    codes_rcp_packed<8>(v, s, w);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 q;
    q.x = w[0];
    q.y = w[1];
    __builtin_amdgcn_raw_buffer_store_b64(q, rq, ok ? (uint32_t)(lr * C + col) : kOob, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rs,
                                          ok && sub == 0 ? (uint32_t)(lr * ngC + col / G) * 2 : kOob, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) tq[(sub * 8 + i) * PB + lr] = (int8_t)(w[i >> 2] >> (8 * (i & 3)));
    if (sub == 0) srow[lr] = s;  // every row group of the tile has the same scale over its 16 lanes
  }
  __syncthreads();

  // ---- columns: lane (c, part) takes column c, rows part * 32 .. + 32
  constexpr int RPT = 32;
  const int c = tid >> 2, part = tid & 3;
  float colv[RPT];
  const uint32_t *qc = (const uint32_t *)(tq + c * PB + part * RPT);
  const float4 *sr = (const float4 *)(srow + part * RPT);
#pragma unroll
  for (int j4 = 0; j4 < RPT / 4; ++j4) {
    const uint32_t qw = qc[j4];
    const float4 sv = sr[j4];
    const float ss[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int b = 0; b < 4; ++b) colv[4 * j4 + b] = (float)(int8_t)(qw >> (8 * b)) * ss[b];
  }
  const uint32_t am = group_max_u32<4>(__builtin_bit_cast(uint32_t, abs_max<RPT>(colv)));
  const float s = group_scale(__builtin_bit_cast(float, am));
  const int64_t gc = c0 + c;
  if (gc >= C) return;
  if (part == 0) scales_t[gc * ngR + by] = scale_bits(s);
  uint32_t w[RPT / 4];
  codes_rcp_packed<RPT>(colv, s, w);
  int8_t *dst = codes_t + gc * R + r0 + part * RPT;
  const int64_t rbase = r0 + part * RPT;
  if (rbase + RPT <= R && (((uintptr_t)dst) & 15) == 0) {
#pragma unroll
    for (int j = 0; j < RPT / 4; j += 4) *(uint4 *)(dst + 4 * j) = make_uint4(w[j], w[j + 1], w[j + 2], w[j + 3]);
  } else {
#pragma unroll
    for (int j = 0; j < RPT; ++j)
      if (rbase + j < R) dst[j] = (int8_t)(w[j / 4] >> (8 * (j % 4)));
  }
}

template <int DT>
__global__ __launch_bounds__(512) void quant_dual_codes_kernel(
    const void *__restrict__ xv, int64_t R, int64_t C, int8_t *__restrict__ codes,
    uint16_t *__restrict__ scales, int8_t *__restrict__ codes_t, uint16_t *__restrict__ scales_t) {
  dual_codes_tile<DT>(xv, R, C, codes, scales, codes_t, scales_t, blockIdx.x, blockIdx.y);
}

// Two X operands (e.g. a layer's weight and its input) in one launch: blocks
// [0, tiles of the first) take the first tensor's 128 x 128 tiles in row-major tile order,
// the rest the second's.
struct DualOperand {
  const void *x;
  int64_t R, C;
  int8_t *codes;
  uint16_t *scales;
  int8_t *codes_t;
  uint16_t *scales_t;
};
template <int DT>
__global__ __launch_bounds__(512) void quant_dual_codes2_kernel(DualOperand a, DualOperand b) {
  const int64_t ta = ((a.C + 127) / 128) * ((a.R + 127) / 128);
  const int64_t i = blockIdx.x;
  const DualOperand &o = i < ta ? a : b;
  const int64_t j = i < ta ? i : i - ta, tc = (o.C + 127) / 128;
  dual_codes_tile<DT>(o.x, o.R, o.C, o.codes, o.scales, o.codes_t, o.scales_t, j % tc, j / tc);
}

// ---------------------------------------------------------------- cross entropy
// Online (max, sum of exp) of one row: the running pair (m, s) absorbs a chunk with maximum
// cm as m' = max(m, cm), s' = s * 2^((m - m') log2 e) + sum 2^((y - m') log2 e). A chunk
// or partner that is entirely -inf contributes nothing (and no inf - inf).
__device__ __forceinline__ void ce_merge(float &m, float &s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  s = (m == -INFINITY ? 0.0f : s * __builtin_amdgcn_exp2f((m - mn) * kLog2e)) +
      (m2 == -INFINITY ? 0.0f : s2 * __builtin_amdgcn_exp2f((m2 - mn) * kLog2e));
  m = mn;
}

// One 256-thread block per row of fp32 logits (R, C): row max, 1 / (sum of exp(y - max))
// and the row's cross-entropy term max + log(sum) - y[t] (0 for an ignored row). A NaN
// anywhere in the row makes its sum NaN, as torch's softmax does.
template <bool VEC>
__global__ __launch_bounds__(256) void ce_row_stats_kernel(
    const float *__restrict__ logits, int64_t C, const int64_t *__restrict__ tgt, int64_t ignore,
    float *__restrict__ rmax, float *__restrict__ rinv, float *__restrict__ rloss) {
  __shared__ float sm[2][4];
  const int64_t row = blockIdx.x;
  const float *y = logits + row * C;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float m = -INFINITY, s = 0.0f;
  bool nan = false;
  auto absorb = [&](const float *v, int n) __attribute__((always_inline)) {
    float cm = -INFINITY;
    for (int i = 0; i < n; ++i) {
      cm = fmaxf(cm, v[i]);
      nan |= v[i] != v[i];
    }
    float cs = 0.0f;
    if (cm != -INFINITY)
      for (int i = 0; i < n; ++i) cs += __builtin_amdgcn_exp2f((v[i] - cm) * kLog2e);
    ce_merge(m, s, cm, cs);
  };
  if (VEC) {  // 16 consecutive elements per chunk (C % 16 == 0, 16-byte aligned rows)
    const float4 *y4 = (const float4 *)y;
    for (int64_t c = (int64_t)tid * 4; c < C / 4; c += 256 * 4) {
      float v[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 q = y4[c + j];
        v[4 * j] = q.x;
        v[4 * j + 1] = q.y;
        v[4 * j + 2] = q.z;
        v[4 * j + 3] = q.w;
      }
      absorb(v, 16);
    }
  } else {
    for (int64_t c = tid; c < C; c += 256) {
      const float v = y[c];
      absorb(&v, 1);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
    ce_merge(m, s, m2, s2);
  }
  nan = __any(nan);
  if (lane == 0) {
    sm[0][wave] = m;
    sm[1][wave] = s;
  }
  __syncthreads();
  if (tid != 0) return;
  m = sm[0][0];
  s = sm[1][0];
  for (int w = 1; w < 4; ++w) ce_merge(m, s, sm[0][w], sm[1][w]);
  if (nan) s = NAN;
  rmax[row] = m;
  rinv[row] = 1.0f / s;
  const int64_t t = tgt[row];
  const bool live = t != ignore && t >= 0 && t < C;
  rloss[row] = live ? (m + logf(s)) - y[t] : 0.0f;
}

// dY of one element per thread (any shape): the fallback when the fused dual path does not
// apply; the codes then come from the dual quantizer run on this dY.
__global__ __launch_bounds__(256) void ce_dy_kernel(const float *__restrict__ logits, int64_t R, int64_t C,
                                                    CeSrc ce) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= R * C) return;
  const int64_t r = idx / C, c = idx % C, t = ce.tgt[r];
  const bool live = t != ce.ignore && t >= 0 && t < C;
  const float e = __builtin_amdgcn_exp2f((logits[idx] - ce.rmax[r]) * kLog2e) * ce.rinv[r];
  ce.dy[idx] = live ? (e - (c == t ? 1.0f : 0.0f)) * *ce.gscale : 0.0f;
}

// ---------------------------------------------------------------- AdamW + requant
// One torch.optim.AdamW step (decoupled weight decay, amsgrad off; the order of
// torch/optim/adam.py _single_tensor_adam, every op one fp32 rounding) on fp32 masters, and
// the int8 codes of the updated masters by the quantize_last_dim contract. The host
// passes torch's python-double scalars rounded to fp32.
struct AdamArgs {
  float decay;      // 1 - lr * weight_decay
  float w1;         // 1 - beta1 (lerp weight)
  float beta2, w2;  // beta2, 1 - beta2
  float eps;
  float step_size;  // lr / (1 - beta1^step)
  float bc2_sqrt;   // (1 - beta2^step)^0.5
};

// A group of 128 consecutive elements of a row per 16 lanes, 8 per lane (gid: the
// (row, group) index of this thread's 16 lanes). VEC: K % 8 == 0 and 16-byte aligned
// buffers, so a lane's 8 elements are all in range or all out.
template <bool VEC>
__device__ __forceinline__ void adamw_group(
    float *__restrict__ p, const float *__restrict__ g, float *__restrict__ m, float *__restrict__ v,
    int64_t rows, int64_t K, int64_t ng, const float *__restrict__ clip, const AdamArgs &a,
    int8_t *__restrict__ codes, uint16_t *__restrict__ scales, int64_t gid) {
  if (gid >= rows * ng) return;  // uniform per 16 lanes
  const int sub = threadIdx.x & 15;
  const int64_t row = gid / ng, grp = gid % ng, col = grp * 128 + sub * 8;
  const int64_t base = row * K + col;
  float pv[8], gv[8], mv[8], vv[8];
  bool ok[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ok[i] = col + i < K;
  if (VEC) {
    if (ok[0]) {
      const float4 *pp = (const float4 *)(p + base), *gp = (const float4 *)(g + base);
      const float4 *mp = (const float4 *)(m + base), *vp = (const float4 *)(v + base);
      const float4 q[8] = {pp[0], pp[1], gp[0], gp[1], mp[0], mp[1], vp[0], vp[1]};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        pv[4 * h] = q[h].x, pv[4 * h + 1] = q[h].y, pv[4 * h + 2] = q[h].z, pv[4 * h + 3] = q[h].w;
        gv[4 * h] = q[2 + h].x, gv[4 * h + 1] = q[2 + h].y, gv[4 * h + 2] = q[2 + h].z, gv[4 * h + 3] = q[2 + h].w;
        mv[4 * h] = q[4 + h].x, mv[4 * h + 1] = q[4 + h].y, mv[4 * h + 2] = q[4 + h].z, mv[4 * h + 3] = q[4 + h].w;
        vv[4 * h] = q[6 + h].x, vv[4 * h + 1] = q[6 + h].y, vv[4 * h + 2] = q[6 + h].z, vv[4 * h + 3] = q[6 + h].w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) pv[i] = gv[i] = mv[i] = vv[i] = 0.0f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pv[i] = ok[i] ? p[base + i] : 0.0f;
      gv[i] = ok[i] ? g[base + i] : 0.0f;
      mv[i] = ok[i] ? m[base + i] : 0.0f;
      vv[i] = ok[i] ? v[base + i] : 0.0f;
    }
  }
  const float c = clip ? *clip : 1.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float gi = clip ? gv[i] * c : gv[i];          // clip_grad_norm_: g.mul_(coef)
    const float pd = pv[i] * a.decay;                    // param.mul_(1 - lr * wd)
    // exp_avg.lerp_(g, 1 - beta1): torch's two forms, switched on the weight (uniform)
    mv[i] = a.w1 < 0.5f ? mv[i] + a.w1 * (gi - mv[i]) : gi - (gi - mv[i]) * (1.0f - a.w1);
    vv[i] = vv[i] * a.beta2 + (a.w2 * gi) * gi;          // exp_avg_sq.mul_(b2).addcmul_(g, g, 1 - b2)
    const float den = sqrtf(vv[i]) / a.bc2_sqrt + a.eps;  // IEEE sqrt and division (build flags)
    pv[i] = pd + (-a.step_size) * (mv[i] / den);         // param.addcdiv_(m, den, -step_size)
    if (!ok[i]) pv[i] = 0.0f;
  }
  if (VEC) {
    if (ok[0]) {
      float4 *pp = (float4 *)(p + base), *mp = (float4 *)(m + base), *vp = (float4 *)(v + base);
      pp[0] = make_float4(pv[0], pv[1], pv[2], pv[3]);
      pp[1] = make_float4(pv[4], pv[5], pv[6], pv[7]);
      mp[0] = make_float4(mv[0], mv[1], mv[2], mv[3]);
      mp[1] = make_float4(mv[4], mv[5], mv[6], mv[7]);
      vp[0] = make_float4(vv[0], vv[1], vv[2], vv[3]);
      vp[1] = make_float4(vv[4], vv[5], vv[6], vv[7]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (ok[i]) {
        p[base + i] = pv[i];
        m[base + i] = mv[i];
        v[base + i] = vv[i];
      }
  }
  if (codes == nullptr) return;  // uniform
  const uint32_t am = group_max_u32<16>(__builtin_bit_cast(uint32_t, abs_max<8>(pv)));
  const float s = group_scale(__builtin_bit_cast(float, am));
  uint32_t w[2];
  codes_rcp_packed<8>(pv, s, w);
  if (sub == 0) scales[row * ng + grp] = scale_bits(s);
  if (VEC) {
    if (ok[0]) *(uint2 *)(codes + base) = make_uint2(w[0], w[1]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (ok[i]) codes[base + i] = (int8_t)(w[i >> 2] >> (8 * (i & 3)));
  }
}

template <bool VEC>
__global__ __launch_bounds__(256) void adamw_requant_kernel(
    float *__restrict__ p, const float *__restrict__ g, float *__restrict__ m, float *__restrict__ v,
    int64_t rows, int64_t K, int64_t ng, const float *__restrict__ clip, AdamArgs a,
    int8_t *__restrict__ codes, uint16_t *__restrict__ scales) {
  adamw_group<VEC>(p, g, m, v, rows, K, ng, clip, a, codes, scales,
                   (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4));
}

// Many masters in one launch: the optimizer step of a whole model is a few launches instead
// of one per parameter (each launch costs the host tens of microseconds). A batch travels
// by value in the kernel arguments; a block finds its master from the prefix of block
// counts with scalar compares.
constexpr int kAdamBatch = 24;
struct AdamTensorArg {
  float *p;
  const float *g;
  float *m, *v;
  int8_t *codes;
  uint16_t *scales;
  int64_t rows, K, ng;
  float step_size, bc2_sqrt;
  int32_t first_block, vec;
};
struct AdamBatchArg {
  AdamTensorArg t[kAdamBatch];
  int32_t n;
};

__global__ __launch_bounds__(256) void adamw_requant_multi_kernel(const AdamBatchArg b,
                                                                 const float *__restrict__ clip,
                                                                 AdamArgs shared) {
  int i = 0;
  for (int k = 1; k < b.n; ++k)
    if (b.t[k].first_block <= (int)blockIdx.x) i = k;
  const AdamTensorArg &t = b.t[i];
  AdamArgs a = shared;
  a.step_size = t.step_size;
  a.bc2_sqrt = t.bc2_sqrt;
  const int64_t gid = (int64_t)((int)blockIdx.x - t.first_block) * 16 + (threadIdx.x >> 4);
  if (t.vec)
    adamw_group<true>(t.p, t.g, t.m, t.v, t.rows, t.K, t.ng, clip, a, t.codes, t.scales, gid);
  else
    adamw_group<false>(t.p, t.g, t.m, t.v, t.rows, t.K, t.ng, clip, a, t.codes, t.scales, gid);
}

template <int SRC>
static int launch_quant_T(const void *x, const uint16_t *in_scales, int64_t nsc_in, int gin,
                          int64_t R, int64_t C, int group, int8_t *codes, uint16_t *scales,
                          hipStream_t st) {
  const int64_t nbc = cdiv(C, 64), ngr = cdiv(R, group);
  const int64_t blocks = nbc * ngr;
  if (blocks > 0x7fffffffLL) return fail(KSD_EINVAL, "quantize_transpose: tensor too large");
  const dim3 g((unsigned)blocks), b(256);
  // 16-byte vector loads need an aligned base and a row pitch that is a multiple of 16 B
  const int esz = SRC == SRC_F32 ? 4 : SRC == SRC_I8 ? 1 : 2;
  const bool rv = ((uintptr_t)x) % 16 == 0 && (C * esz) % 16 == 0;
  switch (group) {
    case 32: quant_T_kernel<SRC, 32><<<g, b, 0, st>>>(x, in_scales, nsc_in, gin, R, C, nbc, ngr, codes, scales, rv); break;
    case 64: quant_T_kernel<SRC, 64><<<g, b, 0, st>>>(x, in_scales, nsc_in, gin, R, C, nbc, ngr, codes, scales, rv); break;
    default: quant_T_kernel<SRC, 128><<<g, b, 0, st>>>(x, in_scales, nsc_in, gin, R, C, nbc, ngr, codes, scales, rv); break;
  }
  return check_launch("quantize_transpose");
}

template <int DT, int G>
static void launch_rows(const void *x, int64_t rows, int64_t K, int64_t stride,
                        int8_t *codes, uint16_t *scales, const float *noise, float d2,
                        bool vec, hipStream_t st) {
  const int64_t ng = cdiv(K, G);
  if (vec && noise == nullptr && K <= (1 << 24)) {
    // four rows per wave where that still gives every CU several blocks
    const unsigned gy = (unsigned)cdiv(K, 512);
    if (cdiv(rows, 16) * gy >= 1024) {
      const dim3 grid((unsigned)cdiv(rows, 16), gy);
      quant_rows_fast_kernel<DT, G, 4><<<grid, 256, 0, st>>>(x, rows, (int)K, stride, (int)ng, codes, scales);
    } else {
      const dim3 grid((unsigned)cdiv(rows, 4), gy);
      quant_rows_fast_kernel<DT, G, 1><<<grid, 256, 0, st>>>(x, rows, (int)K, stride, (int)ng, codes, scales);
    }
    return;
  }
  const int64_t lanes = rows * ng * (G / 8);
  const unsigned blocks = (unsigned)cdiv(lanes, 256);
  if (vec)
    quant_rows_kernel<DT, G, true><<<blocks, 256, 0, st>>>(x, rows, K, stride, ng, codes, scales, noise, d2);
  else
    quant_rows_kernel<DT, G, false><<<blocks, 256, 0, st>>>(x, rows, K, stride, ng, codes, scales, noise, d2);
}

// ----------------------------------------------------------------------------------
// LayerNorm forward (nn.LayerNorm, model/block.py:27-41: ln_attn / ln_ffn) fused with the
// GS128 quantization of its output, the A operand of the Int8Linear that follows
// (linear.py:69 quantize_last_dim). One block per row, ceil(d / 8) lanes rounded up to
// whole waves (d <= 4096: at most 8 waves); lane i holds elements 8i .. 8i + 7, so the 16
// lanes of a 128-element group sit in one wave. mean and the biased variance are fp32,
// two passes: each wave sums its lanes by DPP, and every lane adds the wave totals in
// wave order from LDS, so all lanes hold the same bits. y = (x - mean) * rstd * w + b,
// rounded to x's dtype (torch's LayerNorm output dtype), is quantized exactly as
// quant_rows_kernel does. VEC: d % 8 == 0 and 16-byte aligned rows, weight and bias.
constexpr int kLnMaxD = 4096;

// Sum over the wave's 64 lanes, the same bits in every lane (all lanes active): within
// each row of 16 by DPP (pairs, quads, half-rows, rows: each step adds the partner's
// partial, which holds the same set of lanes), then the four row sums in a fixed order.
__device__ __forceinline__ float ln_wave_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

template <int DT, bool VEC>
__global__ __launch_bounds__(512) void ln_quant_kernel(
    const void *__restrict__ xv, int64_t rows, int d, int64_t stride, const float *__restrict__ w,
    const float *__restrict__ bvec, float eps, int ngroups, int8_t *__restrict__ codes,
    uint16_t *__restrict__ scales, void *__restrict__ y, float *__restrict__ mean_out,
    float *__restrict__ rstd_out) {
  using T = typename Elem<DT>::T;
  __shared__ float red[2][8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const int64_t row = blockIdx.x;
  const int k0 = tid * 8;
  const bool kok = k0 < d;
  const T *xr = (const T *)xv + row * stride;
  float v[8], wv[8], bv[8];
  if (VEC) {
    cvt_raw8<DT>(load_raw8<DT>(xr + (kok ? k0 : 0)), kok, v);
    if (w) cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(w + (kok ? k0 : 0)), kok, wv);
    if (bvec) cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(bvec + (kok ? k0 : 0)), kok, bv);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool ok = k0 + i < d;
      v[i] = ok ? Elem<DT>::load(xr + k0 + i) : 0.0f;
      if (w) wv[i] = ok ? w[k0 + i] : 0.0f;
      if (bvec) bv[i] = ok ? bvec[k0 + i] : 0.0f;
    }
  }
  if (!w) {
#pragma unroll
    for (int i = 0; i < 8; ++i) wv[i] = 1.0f;
  }
  if (!bvec) {
#pragma unroll
    for (int i = 0; i < 8; ++i) bv[i] = 0.0f;
  }
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sum += v[i];
  sum = ln_wave_sum(sum);
  if (lane == 0) red[0][wave] = sum;
  __syncthreads();
  sum = red[0][0];
  for (int i = 1; i < nw; ++i) sum += red[0][i];
  const float mean = sum / (float)d;
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float c = k0 + i < d ? v[i] - mean : 0.0f;
    sq += c * c;
  }
  sq = ln_wave_sum(sq);
  if (lane == 0) red[1][wave] = sq;
  __syncthreads();
  sq = red[1][0];
  for (int i = 1; i < nw; ++i) sq += red[1][i];
  const float rstd = 1.0f / sqrtf(sq / (float)d + eps);
  if (tid == 0) {
    if (mean_out) mean_out[row] = mean;
    if (rstd_out) rstd_out[row] = rstd;
  }
  float yv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    yv[i] = k0 + i < d ? round_to_dt<DT>((v[i] - mean) * rstd * wv[i] + bv[i]) : 0.0f;
  const uint32_t am = __builtin_bit_cast(uint32_t, abs_max<8>(yv));
  const float sc = group_scale(__builtin_bit_cast(float, group_max_u32<16>(am)));
  int8_t *cr = codes + row * d;
  if (VEC && kok) {
    uint32_t qw[2];
    codes_rcp_packed<8>(yv, sc, qw);
    *(uint2 *)(cr + k0) = make_uint2(qw[0], qw[1]);
  } else if (kok) {
    int8_t q[8];
    codes_rcp<8>(yv, sc, q);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < d) cr[k0 + i] = q[i];
  }
  if (kok && (lane & 15) == 0) scales[row * ngroups + (k0 >> 7)] = scale_bits(sc);
  if (y != nullptr && kok) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < d) store_out<DT>(y, row * d + k0 + i, yv[i]);
  }
}

template <int DT>
static void launch_rows_g(int group, const void *x, int64_t rows, int64_t K, int64_t stride,
                          int8_t *codes, uint16_t *scales, const float *noise, float d2,
                          bool vec, hipStream_t st) {
  if (group == 32) launch_rows<DT, 32>(x, rows, K, stride, codes, scales, noise, d2, vec, st);
  else if (group == 64) launch_rows<DT, 64>(x, rows, K, stride, codes, scales, noise, d2, vec, st);
  else launch_rows<DT, 128>(x, rows, K, stride, codes, scales, noise, d2, vec, st);
}

}  // namespace ksd

using namespace ksd;

extern "C" int ksd_quantize_lastdim(const void *x, int x_dtype, int64_t rows, int64_t K,
                                    int64_t x_stride, int group, int8_t *codes,
                                    uint16_t *scales, const float *noise, float dither2,
                                    void *stream) {
  if (!valid_group(group)) return fail(KSD_EINVAL, "group must be 32, 64 or 128, got %d", group);
  if (rows < 0 || K < 0 || x_stride < K) return fail(KSD_EINVAL, "bad quantize shape");
  if (rows == 0 || K == 0) return KSD_OK;
  if (cdiv(rows * cdiv(K, group) * (group / 8), 256) > 0x7fffffffLL)
    return fail(KSD_EINVAL, "quantize: tensor too large");
  hipStream_t st = (hipStream_t)stream;
  const int esz = x_dtype == KSD_F32 ? 4 : 2;
  const bool vec = (((uintptr_t)x) % 16 == 0) && ((x_stride * esz) % 16 == 0) &&
                   (K % 8 == 0) && (((uintptr_t)codes) % 8 == 0);
  switch (x_dtype) {
    case KSD_F32: launch_rows_g<KSD_F32>(group, x, rows, K, x_stride, codes, scales, noise, dither2, vec, st); break;
    case KSD_BF16: launch_rows_g<KSD_BF16>(group, x, rows, K, x_stride, codes, scales, noise, dither2, vec, st); break;
    case KSD_F16: launch_rows_g<KSD_F16>(group, x, rows, K, x_stride, codes, scales, noise, dither2, vec, st); break;
    default: return fail(KSD_ETYPE, "quantize expects float32, bfloat16 or float16 input");
  }
  return check_launch("quantize_lastdim");
}

// ----------------------------------------------------------------------------------
// Int8 embedding gather: out[i, :] = codes[ids[i], :] * scales[ids[i], :/G], the row of a
// per-row GS-quantized table dequantized by token id (exact in fp32, as dequantize). One
// wave per row, 8 elements per lane per pass; an id outside [0, V) gives a zero row (the
// host checks ids before the launch unless told not to).
template <int OUT, bool VEC>
__global__ __launch_bounds__(256) void embed_gather_kernel(
    const int8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const int64_t *__restrict__ ids, int64_t n, int64_t V, int64_t d, int64_t nsc, int group,
    void *__restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const int lane = threadIdx.x & 63;
  const int64_t id = ids[row];
  const bool ok = id >= 0 && id < V;
  const int8_t *src = codes + (ok ? id : 0) * d;
  const uint16_t *sc = scales + (ok ? id : 0) * nsc;
  for (int64_t c0 = (int64_t)lane * 8; c0 < d; c0 += 64 * 8) {
    float v[8];
    if (VEC) {
      const uint2 w = *(const uint2 *)(src + c0);
      const float s = ok ? f16_to_f32(sc[c0 / group]) : 0.0f;  // 8 | group: one scale
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = (float)(int8_t)((j < 4 ? w.x : w.y) >> (8 * (j & 3))) * s;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t c = c0 + j;
        v[j] = (ok && c < d) ? (float)src[c] * f16_to_f32(sc[c / group]) : 0.0f;
      }
    }
    const int64_t base = row * d + c0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (!VEC && c0 + j >= d) break;
      if constexpr (OUT == KSD_F32) ((float *)out)[base + j] = v[j];
      else if constexpr (OUT == KSD_BF16) ((uint16_t *)out)[base + j] = f32_to_bf16(v[j]);
      else ((uint16_t *)out)[base + j] = f16_bits(v[j]);
    }
  }
}

extern "C" int ksd_embedding_gather_int8(const int8_t *codes, const uint16_t *scales,
                                         const int64_t *ids, int64_t n, int64_t V, int64_t d,
                                         int group, void *out, int out_dtype, void *stream) {
  if (!valid_group(group)) return fail(KSD_EINVAL, "embedding_gather: group must be 32, 64 or 128");
  if (n < 0 || V < 0 || d < 0) return fail(KSD_EINVAL, "embedding_gather: negative shape");
  if (n == 0 || d == 0) return KSD_OK;
  if (V == 0) return fail(KSD_EINVAL, "embedding_gather: empty table");
  if (!codes || !scales || !ids || !out) return fail(KSD_EINVAL, "embedding_gather: null pointer");
  if (cdiv(n, 4) > 0x7fffffffLL) return fail(KSD_EINVAL, "embedding_gather: too many rows");
  const int64_t nsc = cdiv(d, group);
  const bool vec = d % 8 == 0 && ((uintptr_t)codes & 7) == 0;
  const dim3 g((unsigned)cdiv(n, 4)), b(256);
  hipStream_t st = (hipStream_t)stream;
#define KSD_EMB(O)                                                                              \
  if (vec) embed_gather_kernel<O, true><<<g, b, 0, st>>>(codes, scales, ids, n, V, d, nsc, group, out); \
  else embed_gather_kernel<O, false><<<g, b, 0, st>>>(codes, scales, ids, n, V, d, nsc, group, out);
  switch (out_dtype) {
    case KSD_F32: KSD_EMB(KSD_F32) break;
    case KSD_BF16: KSD_EMB(KSD_BF16) break;
    case KSD_F16: KSD_EMB(KSD_F16) break;
    default: return fail(KSD_ETYPE, "embedding_gather: unsupported output dtype %d", out_dtype);
  }
#undef KSD_EMB
  return check_launch("embedding_gather_int8");
}

extern "C" int ksd_dequantize_lastdim(const int8_t *codes, const uint16_t *scales,
                                      int64_t rows, int64_t K, int64_t n_scales, int group,
                                      float *out, void *stream) {
  if (group <= 0) return fail(KSD_EINVAL, "dequantize: group must be positive");
  if (rows == 0 || K == 0) return KSD_OK;
  const int64_t n = rows * K;
  if (cdiv(n, 256) > 0x7fffffffLL) return fail(KSD_EINVAL, "dequantize: tensor too large");
  dequant_rows_kernel<<<(unsigned)cdiv(n, 256), 256, 0, (hipStream_t)stream>>>(
      codes, scales, rows, K, n_scales, group, out);
  return check_launch("dequantize_lastdim");
}

extern "C" int ksd_quantize_transpose(const void *x, int x_dtype, int64_t R, int64_t C,
                                      int group, int8_t *codes, uint16_t *scales,
                                      void *stream) {
  if (!valid_group(group)) return fail(KSD_EINVAL, "group must be 32, 64 or 128, got %d", group);
  if (R == 0 || C == 0) return KSD_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (x_dtype) {
    case KSD_F32: return launch_quant_T<SRC_F32>(x, nullptr, 0, 1, R, C, group, codes, scales, st);
    case KSD_BF16: return launch_quant_T<SRC_BF16>(x, nullptr, 0, 1, R, C, group, codes, scales, st);
    case KSD_F16: return launch_quant_T<SRC_F16>(x, nullptr, 0, 1, R, C, group, codes, scales, st);
    default: return fail(KSD_ETYPE, "quantize expects float32, bfloat16 or float16 input");
  }
}

extern "C" int ksd_requant_transpose(const int8_t *codes, const uint16_t *scales, int64_t R,
                                     int64_t C, int group_in, int group, int8_t *out_codes,
                                     uint16_t *out_scales, void *stream) {
  if (!valid_group(group) || !valid_group(group_in))
    return fail(KSD_EINVAL, "group must be 32, 64 or 128");
  if (R == 0 || C == 0) return KSD_OK;
  return launch_quant_T<SRC_I8>(codes, scales, cdiv(C, group_in), group_in, R, C, group, out_codes,
                                out_scales, (hipStream_t)stream);
}

extern "C" int ksd_quantize_dual(const void *x, int x_dtype, int64_t R, int64_t C, int group,
                                 int t_from_codes, int8_t *codes, uint16_t *scales,
                                 int8_t *codes_t, uint16_t *scales_t, void *stream) {
  if (!valid_group(group)) return fail(KSD_EINVAL, "group must be 32, 64 or 128, got %d", group);
  if (R < 0 || C < 0) return fail(KSD_EINVAL, "quantize_dual: negative shape");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "quantize expects float32, bfloat16 or float16 input");
  if (R == 0 || C == 0) return KSD_OK;
  if (!x || !codes || !scales || !codes_t || !scales_t)
    return fail(KSD_EINVAL, "quantize_dual: null pointer");
  if (t_from_codes < 0 || t_from_codes > 2) return fail(KSD_EINVAL, "quantize_dual: mode must be 0, 1 or 2");
  hipStream_t st = (hipStream_t)stream;
  const int esz = x_dtype == KSD_F32 ? 4 : 2;
  const bool fast = group == 128 && C % 8 == 0 && ((uintptr_t)x) % 16 == 0 && (C * esz) % 16 == 0 &&
                    ((uintptr_t)codes) % 8 == 0 && cdiv(R, 128) <= 65535 && cdiv(C, 128) <= 0x7fffffff &&
                    128 * C * 4 <= 0x7fffffffLL;
  if (t_from_codes == 2 && !fast)
    return fail(KSD_EINVAL, "quantize_dual: the fp16 mode needs group 128, C %% 8 == 0 and 16-byte rows");
  if (!fast) {
    // the two single-layout kernels: row codes, then the transposed codes of x or of them
    int rc = ksd_quantize_lastdim(x, x_dtype, R, C, C, group, codes, scales, nullptr, 0.0f, stream);
    if (rc) return rc;
    if (t_from_codes)
      return launch_quant_T<SRC_I8>(codes, scales, cdiv(C, group), group, R, C, group, codes_t, scales_t, st);
    return ksd_quantize_transpose(x, x_dtype, R, C, group, codes_t, scales_t, stream);
  }
  const dim3 grid((unsigned)cdiv(C, 128), (unsigned)cdiv(R, 128));
#define KSD_DUAL(DT)                                                                                      \
  if (t_from_codes == 1)                                                                                  \
    quant_dual_codes_kernel<DT><<<grid, 512, 0, st>>>(x, R, C, codes, scales, codes_t, scales_t);         \
  else if (t_from_codes == 2)                                                                             \
    quant_dual_kernel<DT, false, true><<<grid, 512, 0, st>>>(x, R, C, codes, scales, codes_t, scales_t);  \
  else                                                                                                    \
    quant_dual_kernel<DT><<<grid, 512, 0, st>>>(x, R, C, codes, scales, codes_t, scales_t);
  switch (x_dtype) {
    case KSD_F32: KSD_DUAL(KSD_F32); break;
    case KSD_BF16: KSD_DUAL(KSD_BF16); break;
    default: KSD_DUAL(KSD_F16); break;
  }
#undef KSD_DUAL
  return check_launch("quantize_dual");
}

extern "C" int ksd_quantize_dual2(const void *x0, int64_t R0, int64_t C0, int8_t *codes0,
                                  uint16_t *scales0, int8_t *codes_t0, uint16_t *scales_t0,
                                  const void *x1, int64_t R1, int64_t C1, int8_t *codes1,
                                  uint16_t *scales1, int8_t *codes_t1, uint16_t *scales_t1,
                                  int x_dtype, int group, void *stream) {
  if (group != 128) return fail(KSD_EINVAL, "quantize_dual2: group must be 128, got %d", group);
  if (R0 < 0 || C0 < 0 || R1 < 0 || C1 < 0) return fail(KSD_EINVAL, "quantize_dual2: negative shape");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "quantize expects float32, bfloat16 or float16 input");
  const int esz = x_dtype == KSD_F32 ? 4 : 2;
  auto fast = [&](const void *x, int64_t R, int64_t C, const int8_t *codes) {
    return R > 0 && C > 0 && C % 8 == 0 && ((uintptr_t)x) % 16 == 0 && (C * esz) % 16 == 0 &&
           ((uintptr_t)codes) % 8 == 0 && 128 * C * 4 <= 0x7fffffffLL;
  };
  if (!fast(x0, R0, C0, codes0) || !fast(x1, R1, C1, codes1) ||
      cdiv(C0, 128) * cdiv(R0, 128) + cdiv(C1, 128) * cdiv(R1, 128) > 0x7fffffffLL) {
    int rc = ksd_quantize_dual(x0, x_dtype, R0, C0, group, 1, codes0, scales0, codes_t0, scales_t0, stream);
    if (rc) return rc;
    return ksd_quantize_dual(x1, x_dtype, R1, C1, group, 1, codes1, scales1, codes_t1, scales_t1, stream);
  }
  if (!codes0 || !scales0 || !codes_t0 || !scales_t0 || !codes1 || !scales1 || !codes_t1 || !scales_t1)
    return fail(KSD_EINVAL, "quantize_dual2: null pointer");
  const DualOperand a{x0, R0, C0, codes0, scales0, codes_t0, scales_t0};
  const DualOperand b{x1, R1, C1, codes1, scales1, codes_t1, scales_t1};
  const unsigned nblk = (unsigned)(cdiv(C0, 128) * cdiv(R0, 128) + cdiv(C1, 128) * cdiv(R1, 128));
  hipStream_t st = (hipStream_t)stream;
  switch (x_dtype) {
    case KSD_F32: quant_dual_codes2_kernel<KSD_F32><<<nblk, 512, 0, st>>>(a, b); break;
    case KSD_BF16: quant_dual_codes2_kernel<KSD_BF16><<<nblk, 512, 0, st>>>(a, b); break;
    default: quant_dual_codes2_kernel<KSD_F16><<<nblk, 512, 0, st>>>(a, b); break;
  }
  return check_launch("quantize_dual2");
}

extern "C" int ksd_quantize_dual_colsum(const void *x, int x_dtype, int64_t R, int64_t C, int group,
                                        int8_t *codes, uint16_t *scales, int8_t *codes_t,
                                        uint16_t *scales_t, float *colsum, float *workspace,
                                        int64_t workspace_bytes, void *stream) {
  if (group != 128) return fail(KSD_EINVAL, "quantize_dual_colsum: group must be 128, got %d", group);
  if (R <= 0 || C < 0) return fail(KSD_EINVAL, "quantize_dual_colsum: needs R > 0 and C >= 0");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "quantize expects float32, bfloat16 or float16 input");
  if (C == 0) return KSD_OK;
  if (!x || !codes || !scales || !codes_t || !scales_t || !colsum)
    return fail(KSD_EINVAL, "quantize_dual_colsum: null pointer");
  const int esz = x_dtype == KSD_F32 ? 4 : 2;
  const bool fast = C % 8 == 0 && ((uintptr_t)x) % 16 == 0 && (C * esz) % 16 == 0 &&
                    ((uintptr_t)codes) % 8 == 0 && cdiv(R, 128) <= 65535 && cdiv(C, 128) <= 0x7fffffff &&
                    128 * C * 4 <= 0x7fffffffLL;
  if (!fast) return fail(KSD_EINVAL, "quantize_dual_colsum: needs C %% 8 == 0 and 16-byte aligned rows");
  const int64_t nt = cdiv(R, 128);
  if (!workspace || workspace_bytes < nt * C * 4 || ((uintptr_t)workspace) % 4 != 0)
    return fail(KSD_EINVAL, "quantize_dual_colsum: needs an fp32 workspace of %lld bytes",
                (long long)(nt * C * 4));
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)cdiv(C, 128), (unsigned)nt);
  switch (x_dtype) {
    case KSD_F32: quant_dual_kernel<KSD_F32><<<grid, 512, 0, st>>>(x, R, C, codes, scales, codes_t, scales_t, CeSrc{}, workspace); break;
    case KSD_BF16: quant_dual_kernel<KSD_BF16><<<grid, 512, 0, st>>>(x, R, C, codes, scales, codes_t, scales_t, CeSrc{}, workspace); break;
    default: quant_dual_kernel<KSD_F16><<<grid, 512, 0, st>>>(x, R, C, codes, scales, codes_t, scales_t, CeSrc{}, workspace); break;
  }
  hipLaunchKernelGGL(colsum_finalize_kernel, dim3((unsigned)cdiv(C, 256)), dim3(256), 0, st, workspace, nt, C, colsum);
  return check_launch("quantize_dual_colsum");
}

extern "C" int ksd_ce_row_stats(const float *logits, int64_t R, int64_t C, const int64_t *targets,
                                int64_t ignore_index, float *row_max, float *row_inv_sum,
                                float *row_loss, void *stream) {
  if (R < 0 || C < 0) return fail(KSD_EINVAL, "ce_row_stats: negative shape");
  if (R == 0) return KSD_OK;
  if (C == 0) return fail(KSD_EINVAL, "ce_row_stats: no classes");
  if (!logits || !targets || !row_max || !row_inv_sum || !row_loss)
    return fail(KSD_EINVAL, "ce_row_stats: null pointer");
  if (R > 0x7fffffffLL) return fail(KSD_EINVAL, "ce_row_stats: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const bool vec = C % 16 == 0 && ((uintptr_t)logits) % 16 == 0;
  if (vec)
    ce_row_stats_kernel<true><<<(unsigned)R, 256, 0, st>>>(logits, C, targets, ignore_index, row_max,
                                                          row_inv_sum, row_loss);
  else
    ce_row_stats_kernel<false><<<(unsigned)R, 256, 0, st>>>(logits, C, targets, ignore_index, row_max,
                                                           row_inv_sum, row_loss);
  return check_launch("ce_row_stats");
}

extern "C" int ksd_ce_backward_quant_dual(const float *logits, int64_t R, int64_t C,
                                          const float *row_max, const float *row_inv_sum,
                                          const int64_t *targets, int64_t ignore_index,
                                          const float *grad_scale, int group, int8_t *codes,
                                          uint16_t *scales, int8_t *codes_t, uint16_t *scales_t,
                                          float *dy_out, void *stream) {
  if (group != 128) return fail(KSD_EINVAL, "ce_backward_quant_dual: group must be 128, got %d", group);
  if (R < 0 || C < 0) return fail(KSD_EINVAL, "ce_backward_quant_dual: negative shape");
  if (R == 0 || C == 0) return KSD_OK;
  if (!logits || !row_max || !row_inv_sum || !targets || !grad_scale || !codes || !scales || !codes_t ||
      !scales_t)
    return fail(KSD_EINVAL, "ce_backward_quant_dual: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const CeSrc ce{row_max, row_inv_sum, targets, ignore_index, grad_scale, dy_out};
  const bool fast = C % 8 == 0 && ((uintptr_t)logits) % 16 == 0 && ((uintptr_t)codes) % 8 == 0 &&
                    (dy_out == nullptr || ((uintptr_t)dy_out) % 16 == 0) && cdiv(R, 128) <= 65535 &&
                    cdiv(C, 128) <= 0x7fffffff && 128 * C * 4 <= 0x7fffffffLL;
  if (fast) {
    const dim3 grid((unsigned)cdiv(C, 128), (unsigned)cdiv(R, 128));
    quant_dual_kernel<KSD_F32, true><<<grid, 512, 0, st>>>(logits, R, C, codes, scales, codes_t,
                                                                  scales_t, ce);
    return check_launch("ce_backward_quant_dual");
  }
  // other shapes: dY into dy_out (required here), then the dual quantizer on it
  if (!dy_out) return fail(KSD_EINVAL, "ce_backward_quant_dual: this shape needs dy_out (R x C fp32)");
  if (cdiv(R * C, 256) > 0x7fffffffLL) return fail(KSD_EINVAL, "ce_backward_quant_dual: tensor too large");
  ce_dy_kernel<<<(unsigned)cdiv(R * C, 256), 256, 0, st>>>(logits, R, C, ce);
  const int rc = check_launch("ce_backward_quant_dual (dY)");
  if (rc) return rc;
  return ksd_quantize_dual(dy_out, KSD_F32, R, C, group, 0, codes, scales, codes_t, scales_t, stream);
}

extern "C" int ksd_adamw_requant(float *param, const float *grad, float *exp_avg, float *exp_avg_sq,
                                 int64_t rows, int64_t K, const float *clip_coef, float decay,
                                 float one_minus_beta1, float beta2, float one_minus_beta2, float eps,
                                 float step_size, float bias_correction2_sqrt, int group, int8_t *codes,
                                 uint16_t *scales, void *stream) {
  if (group != 128) return fail(KSD_EINVAL, "adamw_requant: group must be 128, got %d", group);
  if (rows < 0 || K < 0) return fail(KSD_EINVAL, "adamw_requant: negative shape");
  if (rows == 0 || K == 0) return KSD_OK;
  if (!param || !grad || !exp_avg || !exp_avg_sq) return fail(KSD_EINVAL, "adamw_requant: null pointer");
  if ((codes == nullptr) != (scales == nullptr))
    return fail(KSD_EINVAL, "adamw_requant: codes and scales go together");
  const int64_t ng = cdiv(K, 128);
  const int64_t blocks = cdiv(rows * ng, 16);
  if (blocks > 0x7fffffffLL) return fail(KSD_EINVAL, "adamw_requant: tensor too large");
  const AdamArgs a{decay, one_minus_beta1, beta2, one_minus_beta2, eps, step_size, bias_correction2_sqrt};
  auto al = [](const void *q, uintptr_t n) { return ((uintptr_t)q) % n == 0; };
  const bool vec = K % 8 == 0 && al(param, 16) && al(grad, 16) && al(exp_avg, 16) && al(exp_avg_sq, 16) &&
                   (codes == nullptr || al(codes, 8));
  hipStream_t st = (hipStream_t)stream;
  if (vec)
    adamw_requant_kernel<true><<<(unsigned)blocks, 256, 0, st>>>(param, grad, exp_avg, exp_avg_sq, rows, K, ng,
                                                                 clip_coef, a, codes, scales);
  else
    adamw_requant_kernel<false><<<(unsigned)blocks, 256, 0, st>>>(param, grad, exp_avg, exp_avg_sq, rows, K, ng,
                                                                  clip_coef, a, codes, scales);
  return check_launch("adamw_requant");
}

extern "C" int ksd_adamw_requant_multi(const KsdAdamTensor *tensors, int n, const float *clip_coef,
                                       float decay, float one_minus_beta1, float beta2,
                                       float one_minus_beta2, float eps, int group, void *stream) {
  if (group != 128) return fail(KSD_EINVAL, "adamw_requant_multi: group must be 128, got %d", group);
  if (n < 0 || (n > 0 && !tensors)) return fail(KSD_EINVAL, "adamw_requant_multi: bad tensor list");
  auto al = [](const void *q, uintptr_t a) { return ((uintptr_t)q) % a == 0; };
  for (int i = 0; i < n; ++i) {
    const KsdAdamTensor &t = tensors[i];
    if (t.rows < 0 || t.K < 0) return fail(KSD_EINVAL, "adamw_requant_multi: tensor %d: negative shape", i);
    if (t.rows == 0 || t.K == 0) continue;
    if (!t.param || !t.grad || !t.exp_avg || !t.exp_avg_sq)
      return fail(KSD_EINVAL, "adamw_requant_multi: tensor %d: null pointer", i);
    if ((t.codes == nullptr) != (t.scales == nullptr))
      return fail(KSD_EINVAL, "adamw_requant_multi: tensor %d: codes and scales go together", i);
    if (cdiv(t.rows * cdiv(t.K, 128), 16) > 0x3fffffffLL)
      return fail(KSD_EINVAL, "adamw_requant_multi: tensor %d too large", i);
  }
  hipStream_t st = (hipStream_t)stream;
  const AdamArgs shared{decay, one_minus_beta1, beta2, one_minus_beta2, eps, 0.0f, 0.0f};
  AdamBatchArg b;
  b.n = 0;
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (b.n == 0) return KSD_OK;
    adamw_requant_multi_kernel<<<(unsigned)blocks, 256, 0, st>>>(b, clip_coef, shared);
    b.n = 0;
    blocks = 0;
    return check_launch("adamw_requant_multi");
  };
  for (int i = 0; i < n; ++i) {
    const KsdAdamTensor &t = tensors[i];
    if (t.rows == 0 || t.K == 0) continue;
    const int64_t ng = cdiv(t.K, 128), nb = cdiv(t.rows * ng, 16);
    if (b.n == kAdamBatch || blocks + nb > 0x7fffffffLL) {
      const int rc = flush();
      if (rc) return rc;
    }
    AdamTensorArg &a = b.t[b.n++];
    a.p = t.param, a.g = t.grad, a.m = t.exp_avg, a.v = t.exp_avg_sq;
    a.codes = t.codes, a.scales = t.scales;
    a.rows = t.rows, a.K = t.K, a.ng = ng;
    a.step_size = t.step_size, a.bc2_sqrt = t.bias_correction2_sqrt;
    a.first_block = (int32_t)blocks;
    a.vec = t.K % 8 == 0 && al(t.param, 16) && al(t.grad, 16) && al(t.exp_avg, 16) &&
            al(t.exp_avg_sq, 16) && (t.codes == nullptr || al(t.codes, 8));
    blocks += nb;
  }
  return flush();
}

extern "C" int ksd_requant_transpose_multi(const KsdRequantT *list, int n, int group, void *stream) {
  if (group != 128) return fail(KSD_EINVAL, "requant_transpose_multi: group must be 128, got %d", group);
  if (n < 0 || (n > 0 && !list)) return fail(KSD_EINVAL, "requant_transpose_multi: bad list");
  for (int i = 0; i < n; ++i) {
    const KsdRequantT &t = list[i];
    if (t.R < 0 || t.C < 0) return fail(KSD_EINVAL, "requant_transpose_multi: entry %d: negative shape", i);
    if (t.R == 0 || t.C == 0) continue;
    if (!t.codes || !t.scales || !t.codes_t || !t.scales_t)
      return fail(KSD_EINVAL, "requant_transpose_multi: entry %d: null pointer", i);
    if (cdiv(t.C, 64) * cdiv(t.R, 128) > 0x3fffffffLL)
      return fail(KSD_EINVAL, "requant_transpose_multi: entry %d too large", i);
  }
  hipStream_t st = (hipStream_t)stream;
  RqtBatchArg b;
  b.n = 0;
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (b.n == 0) return KSD_OK;
    requant_T_multi_kernel<<<(unsigned)blocks, 256, 0, st>>>(b);
    b.n = 0;
    blocks = 0;
    return check_launch("requant_transpose_multi");
  };
  for (int i = 0; i < n; ++i) {
    const KsdRequantT &t = list[i];
    if (t.R == 0 || t.C == 0) continue;
    const int64_t nbc = cdiv(t.C, 64), ngr = cdiv(t.R, 128), nb = nbc * ngr;
    if (b.n == kRqtBatch || blocks + nb > 0x7fffffffLL) {
      const int rc = flush();
      if (rc) return rc;
    }
    RqtArg &a = b.t[b.n++];
    a.x = t.codes, a.s = t.scales, a.codes = t.codes_t, a.scales = t.scales_t;
    a.R = t.R, a.C = t.C, a.nbc = nbc, a.ngr = ngr;
    a.first_block = (int32_t)blocks;
    a.rv = ((uintptr_t)t.codes) % 16 == 0 && t.C % 16 == 0;
    blocks += nb;
  }
  return flush();
}

extern "C" int ksd_layernorm_quant(const void *x, int x_dtype, int64_t rows, int64_t d,
                                   int64_t x_stride, const float *weight, const float *bias,
                                   float eps, int group, int8_t *codes, uint16_t *scales,
                                   void *y_out, float *mean_out, float *rstd_out, void *stream) {
  if (group != 128) return fail(KSD_EINVAL, "layernorm_quant: group must be 128, got %d", group);
  if (rows < 0 || d < 1 || x_stride < d) return fail(KSD_EINVAL, "layernorm_quant: bad shape");
  if (d > kLnMaxD) return fail(KSD_EINVAL, "layernorm_quant: d above %d is not supported", kLnMaxD);
  if (!(eps >= 0.0f) || eps > 1.0f) return fail(KSD_EINVAL, "layernorm_quant: eps must be in [0, 1]");
  if (rows == 0) return KSD_OK;
  if (!x || !codes || !scales) return fail(KSD_EINVAL, "layernorm_quant: null pointer");
  if (rows > 0x7fffffffLL) return fail(KSD_EINVAL, "layernorm_quant: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const int esz = x_dtype == KSD_F32 ? 4 : 2;
  const bool vec = (((uintptr_t)x) % 16 == 0) && ((x_stride * esz) % 16 == 0) && (d % 8 == 0) &&
                   (((uintptr_t)codes) % 8 == 0);
  const bool v = vec && (((uintptr_t)weight) % 16 == 0) && (((uintptr_t)bias) % 16 == 0);
  const int ng = (int)cdiv(d, 128);
  const int threads = (int)cdiv(cdiv(d, 8), 64) * 64;
  const dim3 grid((unsigned)rows);
#define KSD_LN(DT, V) \
  ln_quant_kernel<DT, V><<<grid, threads, 0, st>>>(x, rows, (int)d, x_stride, weight, bias, eps, ng, codes, scales, y_out, mean_out, rstd_out)
  switch (x_dtype) {
    case KSD_F32: if (v) KSD_LN(KSD_F32, true); else KSD_LN(KSD_F32, false); break;
    case KSD_BF16: if (v) KSD_LN(KSD_BF16, true); else KSD_LN(KSD_BF16, false); break;
    case KSD_F16: if (v) KSD_LN(KSD_F16, true); else KSD_LN(KSD_F16, false); break;
    default: return fail(KSD_ETYPE, "layernorm_quant expects float32, bfloat16 or float16 input");
  }
#undef KSD_LN
  return check_launch("layernorm_quant");
}

extern "C" int ksd_abi_version(void) { return 2; }

extern "C" int ksd_last_error(char *buf, size_t len) {
  if (buf == nullptr || len == 0) return KSD_EINVAL;
  snprintf(buf, len, "%s", ksd::g_err);
  return KSD_OK;
}
