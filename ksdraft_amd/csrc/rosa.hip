// Rosa mixer step kernels for gfx950 (reference ksdraft/model/rosa.py,
// ksdraft/kernels/rosa_credit_gpu.py).
//
//   rosa_shift_quant_kernel  RosaMixer._shifted (rosa.py:128-133) fused with the
//                            quantize_last_dim of each Int8Linear input: one pass over x
//                            emits the int8 codes + fp16 scales of q_in, k_in and v_in.
//   rosa_pack_kernel         (x > 0) bits of (B, T, S) projections, packed per stream
//                            along T into 32-bit words (bit b of word w = position 32w+b).
//   rosa_match_kernel        _match_payload_sign (rosa.py:40-98): per position t the
//                            latest endpoint j < t of the longest common suffix of
//                            q[..t] and k[..j], capped at min(j+1, lmax).
//   rosa_hard_kernel         payload[s] * sign, transposed back to (B, T, S).
//
// The match is a bit-sliced walk over lengths. For a fixed t let A_L be the set of start
// positions j' whose key window k[j'..j'+L-1] equals q[t-L+1..t]; then
//     A_1 = { j' <= t-1 : k[j'] == q[t] },   A_{L+1}(j') = A_L(j'+1) & (k[j'] == q[t-L]),
// one funnel shift and two bitwise ops per 32 candidates per length. A candidate j = j'+L-1
// survives to length L exactly when its (capped) common suffix is >= L, so the last
// non-empty length is the best length and its highest surviving j the latest endpoint.
// Candidates are walked in chunks of kCH words; each chunk carries two words of halo to
// its left so every chain j'..j'+61 of its own candidates lies inside the chunk.
#include <stdlib.h>
#include <string.h>
#include <type_traits>

#include "ksd_common.h"

namespace ksd {

// ---------------------------------------------------------------- shift + quantize

// Load 8 consecutive features of a row as fp32 (k0 + 8 <= d on the vector path).
template <int DT, bool VEC>
__device__ __forceinline__ void load8(const typename Elem<DT>::T *p, int k0, int d, bool ok, float *v) {
  if (VEC && ok) {
    if constexpr (DT == KSD_F32) {
      const float4 a = *(const float4 *)(p + k0), b = *(const float4 *)(p + k0 + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const uint4 a = *(const uint4 *)(p + k0);
      const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
        v[2 * i] = Elem<DT>::load(&lo);
        v[2 * i + 1] = Elem<DT>::load(&hi);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = ok && k0 + i < d ? Elem<DT>::load(p + k0 + i) : 0.0f;
  }
}

// Block = 4 waves x 64 lanes; a wave walks RT consecutive rows (tokens) and a lane owns 8
// consecutive features, so a group is G/8 adjacent lanes of one wave (grid.y walks the row
// in 512-feature slices). Each row is read once: it is the next row's previous token, and
// the row after it is loaded (unconditionally, from a clamped valid address) while the
// current one is encoded. q_in = prev + (x - prev) * sigmoid(mix): x - prev is an op in
// x's dtype (rounded to it), the rest is fp32 (torch promotes the bf16/fp16 tensor against
// the fp32 sigmoid). VEC: d % 8 == 0 and every row, sigmoid and code row 16/8-byte aligned.
template <int DT, int G, bool VEC, int RT>
__global__ void __launch_bounds__(256) rosa_shift_quant_kernel(
    const void *__restrict__ x, int rows, int T, int d,
    const float *__restrict__ sig_q, const float *__restrict__ sig_k, const float *__restrict__ sig_v,
    int8_t *__restrict__ cq, uint16_t *__restrict__ sq, int8_t *__restrict__ ck,
    uint16_t *__restrict__ sk, int8_t *__restrict__ cv, uint16_t *__restrict__ sv, int ngroups) {
  using E = Elem<DT>;
  constexpr int LPG = G / 8;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = ((int)blockIdx.x * 4 + wave) * RT;
  if (row0 >= rows) return;                                   // wave-uniform
  const int k0 = ((int)blockIdx.y * 64 + (int)(threadIdx.x & 63)) * 8;
  const bool kok = k0 < d;
  const int kc = kok ? k0 : 0;                                // a valid column for every lane
  float sg[3][8];
  const typename E::T *xb = (const typename E::T *)x + kc;
  if constexpr (VEC) {
    cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(sig_q + kc), kok, sg[0]);
    cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(sig_k + kc), kok, sg[1]);
    cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(sig_v + kc), kok, sg[2]);
  } else {
    load8<KSD_F32, false>(sig_q, k0, d, kok, sg[0]);
    load8<KSD_F32, false>(sig_k, k0, d, kok, sg[1]);
    load8<KSD_F32, false>(sig_v, k0, d, kok, sg[2]);
  }
  int8_t *codes[3] = {cq, ck, cv};
  uint16_t *scales[3] = {sq, sk, sv};
  int t = row0 % T;
  float xv[8], pv[8];
  Raw8<DT> rn;
  if constexpr (VEC) {
    Raw8<DT> rp = load_raw8<DT>(xb + (int64_t)(row0 > 0 ? row0 - 1 : 0) * d);
    rn = load_raw8<DT>(xb + (int64_t)row0 * d);
    cvt_raw8<DT>(rp, kok && t > 0, pv);
  } else {
    const typename E::T *xr = (const typename E::T *)x + (int64_t)row0 * d;
    load8<DT, false>(xr - d, k0, d, kok && t > 0, pv);
  }
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int row = row0 + i;
    if (row >= rows) break;                                   // wave-uniform
    if constexpr (VEC) {
      cvt_raw8<DT>(rn, kok, xv);
      if (i + 1 < RT) rn = load_raw8<DT>(xb + (int64_t)min(row + 1, rows - 1) * d);
    } else {
      load8<DT, false>((const typename E::T *)x + (int64_t)row * d, k0, d, kok, xv);
    }
    if (t == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = 0.0f;
    }
    float diff[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) diff[e] = xv[e] - pv[e];
    if constexpr (DT == KSD_BF16) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) bf16_round2(diff[e], diff[e + 1]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) diff[e] = round_to_dt<DT>(diff[e]);
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = pv[e] + diff[e] * sg[m][e];
      const uint32_t am = __builtin_bit_cast(uint32_t, abs_max<8>(v));
      const float s = group_scale(__builtin_bit_cast(float, group_max_u32<LPG>(am)));
      if constexpr (VEC) {
        // stores without branches: a lane past d (or not leading its group, for the
        // scale) gets an offset past num_records, and the buffer unit drops its store
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        u32x2 q;
        uint32_t qw[2];
        codes_rcp_packed<8>(v, s, qw);
        q.x = qw[0];
        q.y = qw[1];
        const auto rc = rsrc(codes[m] + (int64_t)row * d, d);
        __builtin_amdgcn_raw_buffer_store_b64(q, rc, kok ? (uint32_t)k0 : kOob, 0, 0);
        const auto rs = rsrc(scales[m] + (int64_t)row * ngroups, 2 * (int64_t)ngroups);
        const bool lead = kok && (k0 / 8) % LPG == 0;
        __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rs, lead ? (uint32_t)(k0 / G) * 2 : kOob, 0, 0);
      } else if (kok) {
        int8_t q[8];
        codes_rcp<8>(v, s, q);
        int8_t *cr = codes[m] + (int64_t)row * d;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (k0 + e < d) cr[k0 + e] = q[e];
        if ((k0 / 8) % LPG == 0) scales[m][(int64_t)row * ngroups + k0 / G] = scale_bits(s);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = xv[e];
    t = t + 1 == T ? 0 : t + 1;
  }
}

// ---------------------------------------------------------------- shift + dual quantize
// Training form of rosa_shift_quant_kernel, group 128. One pass over a 128 x 128 tile of x
// (rows = tokens, columns = features) emits, for each of q_in, k_in and v_in, the row codes
// of the forward GEMM and the operand dW needs: X^T requantized along the tokens from those
// row codes, the double-quant recipe quant(dequant(quant(X))^T) (ks3_int8.py:417-420) that
// the Int8Linear training forward applies to its input. The row phase is
// quant_dual_codes_kernel's, with each shifted value formed on load from x[r] and x[r - 1]
// (0 at the first token of a sequence) exactly as rosa_shift_quant_kernel forms it; the three
// tiles of row codes (column-major, 132-byte pitch) and row scales then go through LDS to
// the column phase. Requires C % 8 == 0 and 16-byte aligned rows.
struct ShiftDualOut {
  int8_t *codes[3];
  uint16_t *scales[3];
  int8_t *codes_t[3];
  uint16_t *scales_t[3];
};

template <int DT>
__global__ __launch_bounds__(512) void rosa_shift_dual_kernel(
    const void *__restrict__ xv, int R, int C, int T, const float *__restrict__ sig_q,
    const float *__restrict__ sig_k, const float *__restrict__ sig_v, ShiftDualOut out) {
  using E = Elem<DT>;
  constexpr int G = 128, PB = 132;
  __shared__ __attribute__((aligned(16))) int8_t tq[3][128 * PB];  // [m][column][row]
  __shared__ __attribute__((aligned(16))) float srow[3][128];
  const int tid = threadIdx.x;
  const int c0 = (int)blockIdx.x * 128, r0 = (int)blockIdx.y * 128;
  const int ngC = (C + G - 1) / G, ngR = (R + G - 1) / G;

  // ---- rows: lane (rr, sub) takes rows r0 + 32 p + rr (p = 0..3), columns c0 + 8 sub .. + 8
  const int rr = tid >> 4, sub = tid & 15;
  const int col = c0 + sub * 8;
  const bool cok = col < C;
  const int cc = cok ? col : 0;
  const typename E::T *xb = (const typename E::T *)xv + cc;
  float sg[3][8];
  cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(sig_q + cc), cok, sg[0]);
  cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(sig_k + cc), cok, sg[1]);
  cvt_raw8<KSD_F32>(load_raw8<KSD_F32>(sig_v + cc), cok, sg[2]);
  const int64_t nrows = min(128, R - r0);
  __amdgpu_buffer_rsrc_t rq[3], rsc[3];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    rq[m] = rsrc(out.codes[m] + (int64_t)r0 * C, nrows * C);
    rsc[m] = rsrc(out.scales[m] + (int64_t)r0 * ngC, 2 * nrows * ngC);
  }
  Raw8<DT> raw[4], rawp[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int rs = min(r0 + 32 * p + rr, R - 1);
    raw[p] = load_raw8<DT>(xb + (int64_t)rs * C);
    rawp[p] = load_raw8<DT>(xb + (int64_t)(rs > 0 ? rs - 1 : 0) * C);
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int lr = 32 * p + rr;
    const int row = r0 + lr;
    const bool ok = cok && row < R;
    float xr[8], pv[8], diff[8];
    cvt_raw8<DT>(raw[p], ok, xr);
    cvt_raw8<DT>(rawp[p], ok && row % T != 0, pv);
#pragma unroll
    for (int e = 0; e < 8; ++e) diff[e] = xr[e] - pv[e];
    if constexpr (DT == KSD_BF16) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) bf16_round2(diff[e], diff[e + 1]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) diff[e] = round_to_dt<DT>(diff[e]);
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = pv[e] + diff[e] * sg[m][e];
      const uint32_t am = group_max_u32<16>(__builtin_bit_cast(uint32_t, abs_max<8>(v)));
      const float s = group_scale(__builtin_bit_cast(float, am));
      uint32_t w[2];
      codes_rcp_packed<8>(v, s, w);
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      u32x2 q;
      q.x = w[0];
      q.y = w[1];
      // one descriptor per tile (a per-lane base would make the compiler loop over the
      // distinct descriptors of a wave around every store); the lane's row is in the offset
      __builtin_amdgcn_raw_buffer_store_b64(q, rq[m], ok ? (uint32_t)(lr * C + col) : kOob, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b16(scale_bits(s), rsc[m],
                                            ok && sub == 0 ? (uint32_t)(lr * ngC + col / G) * 2 : kOob, 0, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i) tq[m][(sub * 8 + i) * PB + lr] = (int8_t)(w[i >> 2] >> (8 * (i & 3)));
      if (sub == 0) srow[m][lr] = s;  // the 16 lanes of a row group share its scale
    }
  }
  __syncthreads();

  // ---- columns: lane (c, part) takes column c, rows part * 32 .. + 32, of each tile
  constexpr int RPT = 32;
  const int c = tid >> 2, part = tid & 3;
  const int gc = c0 + c;
  const int rbase = r0 + part * RPT;
#pragma unroll
  for (int m = 0; m < 3; ++m) {  // unrolled: `out` is indexed by constants only
    float colv[RPT];
    const uint32_t *qc = (const uint32_t *)(tq[m] + c * PB + part * RPT);
    const float4 *sr = (const float4 *)(srow[m] + part * RPT);
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
    uint32_t w[RPT / 4];
    codes_rcp_packed<RPT>(colv, s, w);
    if (gc < C) {
      if (part == 0) out.scales_t[m][(int64_t)gc * ngR + blockIdx.y] = scale_bits(s);
      int8_t *dst = out.codes_t[m] + (int64_t)gc * R + rbase;
      if (rbase + RPT <= R && (((uintptr_t)dst) & 15) == 0) {
#pragma unroll
        for (int j = 0; j < RPT / 4; j += 4) *(uint4 *)(dst + 4 * j) = make_uint4(w[j], w[j + 1], w[j + 2], w[j + 3]);
      } else {
#pragma unroll
        for (int j = 0; j < RPT; ++j)
          if (rbase + j < R) dst[j] = (int8_t)(w[j / 4] >> (8 * (j % 4)));
      }
    }
  }
}

// Backward of the time shift, q_in = prev + (x - prev) * s_q (and k, v; rosa.py:128-133),
// given the three input gradients g_q, g_k, g_v (fp32, the projections' dX):
//   dx[r]   = sum_m g_m[r] * s_m + [r + 1 in r's sequence] (g_m[r+1] - g_m[r+1] * s_m)
//   ds_m[c] = sum_r g_m[r, c] * (x[r, c] - prev[r, c])    (the gradient of sigmoid(mix_m))
// with x - prev rounded to x's dtype as in the forward and dx stored in x's dtype. A block is
// 4 waves; a lane owns 4 consecutive features and wave w walks its RB rows downward, so
// g_m[r + 1] and x[r] come from the previous iteration. The block's ds sums (its 4 waves
// added in order) go to ds_part (row block, 3, C); the caller adds the row blocks. The grid
// is (ceil(C / 256), ceil(R / (4 RB))).
template <int DT, int RB, bool VEC>
__global__ __launch_bounds__(256) void rosa_shift_bwd_kernel(
    const void *__restrict__ xv, const float *__restrict__ gq, const float *__restrict__ gk,
    const float *__restrict__ gv, const float *__restrict__ sig_q, const float *__restrict__ sig_k,
    const float *__restrict__ sig_v, int R, int C, int T, void *__restrict__ dx,
    float *__restrict__ ds_part) {
  using E = Elem<DT>;
  __shared__ float red[4][3][256];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = ((int)blockIdx.x * 64 + lane) * 4;
  const bool cok = c < C;
  const float *g[3] = {gq, gk, gv};
  const float *sp[3] = {sig_q, sig_k, sig_v};
  auto ld4 = [&](const float *p, int row, bool ok, float *v) {
    if (VEC) {
      const float4 a = ok ? *(const float4 *)(p + (int64_t)row * C + c) : float4{0.f, 0.f, 0.f, 0.f};
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = ok && c + i < C ? p[(int64_t)row * C + c + i] : 0.0f;
    }
  };
  auto ldx4 = [&](int row, bool ok, float *v) {
    const typename E::T *p = (const typename E::T *)xv + (int64_t)row * C + c;
    if constexpr (VEC && DT == KSD_F32) {
      ld4((const float *)xv, row, ok, v);
    } else if constexpr (VEC) {
      uint2 a = ok ? *(const uint2 *)p : uint2{0u, 0u};
      const uint16_t h[4] = {(uint16_t)(a.x & 0xffffu), (uint16_t)(a.x >> 16), (uint16_t)(a.y & 0xffffu),
                             (uint16_t)(a.y >> 16)};
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = ok ? E::load(&h[i]) : 0.0f;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = ok && c + i < C ? E::load(p + i) : 0.0f;
    }
  };
  float s[3][4], ds[3][4], gn[3][4];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    ld4(sp[m], 0, cok, s[m]);
#pragma unroll
    for (int i = 0; i < 4; ++i) ds[m][i] = 0.0f;
  }
  const int lo = (int)blockIdx.y * 4 * RB + wave * RB;
  const int hi = min(lo + RB, R) - 1;  // rows lo..hi, walked downward
  if (lo <= hi) {
    // the row after hi contributes its prev-term when it continues hi's sequence
    const bool nxt = hi + 1 < R && (hi + 1) % T != 0;
#pragma unroll
    for (int m = 0; m < 3; ++m) ld4(g[m], hi + 1, cok && nxt, gn[m]);
    float xr[4];
    ldx4(hi, cok, xr);
    for (int r = hi; r >= lo; --r) {
      const bool has_prev = r % T != 0;
      float xp[4], diff[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
      ldx4(r > 0 ? r - 1 : 0, cok && r > 0, xp);
#pragma unroll
      for (int i = 0; i < 4; ++i) diff[i] = round_to_dt<DT>(xr[i] - (has_prev ? xp[i] : 0.0f));
#pragma unroll
      for (int m = 0; m < 3; ++m) {
        float gr[4];
        ld4(g[m], r, cok, gr);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i] += gr[i] * s[m][i];
          acc[i] += gn[m][i] - gn[m][i] * s[m][i];
          ds[m][i] += gr[i] * diff[i];
          gn[m][i] = has_prev ? gr[i] : 0.0f;
        }
      }
      if (cok) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (VEC || c + i < C) store_out<DT>(dx, (int64_t)r * C + c + i, acc[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) xr[i] = xp[i];
    }
  }
#pragma unroll
  for (int m = 0; m < 3; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][m][lane * 4 + i] = ds[m][i];
  __syncthreads();
  // 768 sums per block (3 x 256 features), 256 threads: 3 each, the waves added in order
  const int f = (int)threadIdx.x, cf = (int)blockIdx.x * 256 + f;
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    const float v = ((red[0][m][f] + red[1][m][f]) + red[2][m][f]) + red[3][m][f];
    if (cf < C) ds_part[((int64_t)blockIdx.y * 3 + m) * C + cf] = v;
  }
}

// ---------------------------------------------------------------- bit packing
// (B, T, S) -> words (B, S, W): one thread per (stream s, word w).
// Up to three projections of one shape in one launch: blockIdx.z = which * B + b.
struct PackSrc {
  const void *x[3];
  uint32_t *bits[3];
};
template <int DT>
__global__ void __launch_bounds__(256) rosa_pack_kernel(PackSrc ps, int64_t B, int64_t T,
                                                        int64_t S, int64_t W) {
  using E = Elem<DT>;
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t w = blockIdx.y, which = blockIdx.z / B, b = blockIdx.z % B;
  if (s >= S) return;
  const void *x = which == 0 ? ps.x[0] : which == 1 ? ps.x[1] : ps.x[2];
  uint32_t *bits = which == 0 ? ps.bits[0] : which == 1 ? ps.bits[1] : ps.bits[2];
  const typename E::T *xb = (const typename E::T *)x + b * T * S + s;
  // all 32 loads first (rows past T clamped to a valid row and masked below)
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = E::load(xb + min(w * 32 + i, T - 1) * S);
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i)
    if (w * 32 + i < T && v[i] > 0.0f) word |= 1u << i;
  bits[(b * S + s) * W + w] = word;
}

// ---------------------------------------------------------------- match
constexpr int kCH = 8;   // candidate words per chunk
constexpr int kStep = 4;  // match lengths per step of the walk

// 64 q bits ending at t in memory order: bit 63 = q[t], bit 63-i = q[t-i] (0 before 0).
__device__ __forceinline__ uint64_t q_window(const uint32_t *qw, int t) {
  const int w = t >> 5, b = t & 31;
  // every load in bounds and none behind a branch, so the three are in flight together
  const uint64_t hi = qw[w];
  const uint64_t mid = qw[max(w - 1, 0)] & (w >= 1 ? ~0u : 0u);
  const uint64_t lo = qw[max(w - 2, 0)] & (w >= 2 ? ~0u : 0u);
  const uint64_t m64 = (hi << 32) | mid;
  return (m64 << (31 - b)) | (b == 31 ? 0ull : (lo >> (b + 1)));
}

// N length steps of a chunk at once (N = 1, 2, 4): from A_L,
//   A_{L+N}(j') = A_L(j'+N) & AND_{i<N} (k[j'+N-1-i] == q[t-L-i]),
// since one step is A_{L+1}(j') = A_L(j'+1) & (k[j'] == q[t-L]). ks[d] holds k shifted
// down by d bits (bit j' of ks[d] = k[j'+d]; zeros past the chunk's top word, where every
// A bit is zero). qs has q[t-L-i] at bit 63-i. The words cover kCH + 2 words; the top
// word's right neighbour is empty. NEG: the chunk starts at word 0, so its two halo words
// lie before position 0 and stay empty. Returns the OR of the new words.
template <bool NEG, int N>
__device__ __forceinline__ uint32_t match_steps(const uint32_t *src, uint32_t *dst,
                                                const uint32_t (&ks)[kStep][kCH + 2], uint64_t qs) {
  uint32_t sm[N];
#pragma unroll
  for (int i = 0; i < N; ++i) sm[i] = (uint32_t)((int32_t)(uint32_t)((qs << i) >> 32) >> 31);
  uint32_t a2 = 0;
#pragma unroll
  for (int c = 0; c < kCH + 2; ++c) {
    const uint32_t right = c + 1 < kCH + 2 ? src[c + 1] : 0u;
    uint32_t v = __builtin_amdgcn_alignbit(right, src[c], N);
#pragma unroll
    for (int i = 0; i < N; ++i) v &= ~(ks[N - 1 - i][c] ^ sm[i]);
    if (NEG && c < 2) v = 0u;
    dst[c] = v;
    a2 |= v;
  }
  return a2;
}

// The length walk of one chunk from A = A_1: returns the last non-empty length L (< lmax
// or = lmax) with A = A_L. Four lengths per step while they fit under lmax and leave a
// survivor; then one two-length and one one-length step find L among the last four.
template <bool NEG>
__device__ __forceinline__ int match_walk(uint32_t *A, const uint32_t (&ks)[kStep][kCH + 2], uint64_t qwin,
                                          int lmax) {
  uint32_t B[kCH + 2];
  uint64_t qs = qwin << 1;  // bit 63 = q[t - L] for the next length step
  int L = 1;
  for (;;) {
    if (L + kStep > lmax || !match_steps<NEG, kStep>(A, B, ks, qs)) break;
    qs <<= kStep;
    L += kStep;
    if (L + kStep > lmax || !match_steps<NEG, kStep>(B, A, ks, qs)) {
#pragma unroll
      for (int c = 0; c < kCH + 2; ++c) A[c] = B[c];
      break;
    }
    qs <<= kStep;
    L += kStep;
  }
  // A = A_L and A_{L+4} is empty (or past lmax): L* lies in [L, L + 3]; a two-length and
  // a one-length step find it
  if (L + 2 <= lmax && match_steps<NEG, 2>(A, B, ks, qs)) {
#pragma unroll
    for (int c = 0; c < kCH + 2; ++c) A[c] = B[c];
    qs <<= 2;
    L += 2;
  }
  if (L + 1 <= lmax && match_steps<NEG, 1>(A, B, ks, qs)) {
#pragma unroll
    for (int c = 0; c < kCH + 2; ++c) A[c] = B[c];
    L += 1;
  }
  return L;
}

// Best (length, endpoint) for position t >= 1. Returns length (0 = no match), sets *jout.
// Chunks are walked from the latest candidates down; a later (older) chunk can only win with
// a strictly longer match, so its survivors are located only when it has one.
__device__ int match_one(const uint32_t *qw, const uint32_t *kw_all, int W, int t, int lmax,
                         int *jout) {
  const uint64_t qwin = q_window(qw, t);
  const int nw = (t - 1) / 32 + 1;  // words holding candidates j in [0, t-1]
  const uint32_t nq0 = ((qwin >> 63) & 1) ? 0u : ~0u;  // k ^ nq == (k == q bit)
  int best_l = 0, best_j = -1;
  for (int w0 = ((nw - 1) / kCH) * kCH; w0 >= 0; w0 -= kCH) {
    if (min(lmax, 32 * (w0 + kCH)) <= best_l) break;  // cannot beat a later endpoint
    uint32_t kw[kCH + 2], A[kCH + 2];
    uint32_t any = 0;
    if (w0 >= 2 && 32 * (w0 + kCH) <= t) {
      // every word of the chunk lies in [0, t-1]: no validity masks
#pragma unroll
      for (int c = 0; c < kCH + 2; ++c) {
        kw[c] = kw_all[w0 - 2 + c];
        A[c] = kw[c] ^ nq0;
        any |= A[c];
      }
    } else {
#pragma unroll
      for (int c = 0; c < kCH + 2; ++c) {
        const int w = w0 - 2 + c;
        const uint32_t kv = kw_all[min(max(w, 0), W - 1)];  // clamped read, masked below
        kw[c] = (w >= 0 && w < W) ? kv : 0u;
        const int hi = t - 1 - 32 * w;  // last valid candidate bit in this word
        const uint32_t valid = w < 0 || hi < 0 ? 0u : (hi >= 31 ? ~0u : (2u << hi) - 1u);
        A[c] = (kw[c] ^ nq0) & valid;
        any |= A[c];
      }
    }
    if (!any) continue;
    uint32_t ks[kStep][kCH + 2];
#pragma unroll
    for (int c = 0; c < kCH + 2; ++c) {
      const uint32_t right = c + 1 < kCH + 2 ? kw[c + 1] : 0u;
      ks[0][c] = kw[c];
#pragma unroll
      for (int d = 1; d < kStep; ++d) ks[d][c] = __builtin_amdgcn_alignbit(right, kw[c], d);
    }
    const int L = w0 >= 2 ? match_walk<false>(A, ks, qwin, lmax) : match_walk<true>(A, ks, qwin, lmax);
    if (L <= best_l) continue;
    // survivors at length L: the highest j = j' + L - 1 with j >= 32 w0 (the halo words' own
    // candidates belong to the older chunk; j < 32 (w0 + kCH) holds for every survivor, as
    // the top word has no right neighbour). In the halo, j >= 32 w0 keeps bits >= 65 - L
    // of word 0 and bits >= 33 - L of word 1.
    const int b0 = 65 - L;
    const uint32_t m0 = b0 >= 32 ? 0u : (~0u << b0);
    const uint32_t m1 = b0 <= 32 ? ~0u : (b0 >= 64 ? 0u : (~0u << (b0 - 32)));
    int fc = -1;
    uint32_t fm = 0u;
#pragma unroll
    for (int c = 0; c < kCH + 2; ++c) {
      const uint32_t m = c == 0 ? (A[0] & m0) : c == 1 ? (A[1] & m1) : A[c];
      if (m) {
        fc = c;
        fm = m;
      }
    }
    if (fc >= 0) {
      best_l = L;
      best_j = 32 * (w0 - 2 + fc) + L - 1 + 31 - (int)__clz(fm);
    }
  }
  *jout = best_j;
  return best_l;
}

// One block per (stream, 256 consecutive positions), a thread per position. The blocks
// of the latest positions (the most candidates) come first in the grid, so the hardware's
// in-order dispatch to free slots balances streams of unequal cost (long-run streams walk
// more lengths) and leaves the cheap early positions for the end. sign (streams, T) int8
// +-1; match_j (streams, T) int32 or NULL.
constexpr int kMatchChunk = 256;
__global__ void __launch_bounds__(kMatchChunk) rosa_match_kernel(const uint32_t *__restrict__ qb,
                                                                 const uint32_t *__restrict__ kb,
                                                                 const uint32_t *__restrict__ vb, int T,
                                                                 int W, int lmax, int nstreams, int nchunks,
                                                                 int8_t *__restrict__ sign,
                                                                 int32_t *__restrict__ match_j) {
  extern __shared__ uint32_t sm[];
  uint32_t *qw = sm, *kw = sm + W, *vw = sm + 2 * W;
  const int64_t item = blockIdx.x;
  const int chunk = nchunks - 1 - (int)(item / nstreams);
  const int64_t s = item % nstreams;
  for (int i = threadIdx.x; i < W; i += kMatchChunk) {
    qw[i] = qb[s * W + i];
    kw[i] = kb[s * W + i];
    vw[i] = vb[s * W + i];
  }
  __syncthreads();
  const int t = chunk * kMatchChunk + threadIdx.x;
  if (t >= T) return;
  int j = -1, L = 0;
  if (t >= 1 && lmax >= 1) L = match_one(qw, kw, W, t, lmax, &j);
  int8_t sg = -1;
  if (L >= 1) sg = ((vw[(j + 1) >> 5] >> ((j + 1) & 31)) & 1u) ? 1 : -1;
  sign[s * T + t] = sg;
  if (match_j) match_j[s * T + t] = L >= 1 ? j : -1;
}

// (B, S, T) int8 sign -> (B, T, S) payload[s] * sign in the output dtype, via a 64x64 tile:
// a thread loads 4 positions of a stream as one word (four streams per thread) and stores
// 4 consecutive streams of a position (16 bytes for fp32, 8 for 16-bit outputs).
template <int DT>
__global__ void __launch_bounds__(256) rosa_hard_kernel(const int8_t *__restrict__ sign,
                                                        const float *__restrict__ payload,
                                                        int64_t T, int64_t S, void *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) int8_t tile[64][68];  // [stream][position]
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * 64, s0 = (int64_t)blockIdx.y * 64;
  const int r = threadIdx.x >> 4, c = threadIdx.x & 15;
  const bool vec_in = (T & 3) == 0 && t0 + 64 <= T;  // whole aligned words of the tile
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int sl = r + 16 * p;
    const int64_t s = s0 + sl, t = t0 + 4 * c;
    uint32_t w = 0u;
    if (s < S) {
      const int8_t *src = sign + (b * S + s) * T + t;
      if (vec_in) {
        w = *(const uint32_t *)src;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (t + j < T) w |= (uint32_t)(uint8_t)src[j] << (8 * j);
      }
    }
    *(uint32_t *)&tile[sl][4 * c] = w;
  }
  __syncthreads();
  float pay[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) pay[j] = s0 + 4 * c + j < S ? payload[s0 + 4 * c + j] : 0.0f;
  const bool vec_out = (S & 3) == 0 && s0 + 4 * c + 4 <= S;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int tl = r + 16 * p;
    const int64_t t = t0 + tl;
    if (t >= T) continue;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = pay[j] * (float)tile[4 * c + j][tl];
    const int64_t o = (b * T + t) * S + s0 + 4 * c;
    if (vec_out) {
      if constexpr (DT == KSD_F32) {
        *(float4 *)((float *)out + o) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        uint16_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = DT == KSD_BF16 ? f32_to_bf16(v[j]) : f16_bits(v[j]);
        *(uint2 *)((uint16_t *)out + o) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (s0 + 4 * c + j < S) store_out<DT>(out, o + j, v[j]);
    }
  }
}


}  // namespace ksd

using namespace ksd;

extern "C" int ksd_rosa_shift_quant(const void *x, int x_dtype, int64_t B, int64_t T, int64_t d,
                                    const float *sig_q, const float *sig_k, const float *sig_v,
                                    int group, int8_t *q_codes, uint16_t *q_scales, int8_t *k_codes,
                                    uint16_t *k_scales, int8_t *v_codes, uint16_t *v_scales,
                                    void *stream) {
  if (B < 0 || T < 0 || d < 0) return fail(KSD_EINVAL, "rosa_shift_quant: negative shape");
  if (!valid_group(group)) return fail(KSD_EINVAL, "rosa_shift_quant: group must be 32, 64 or 128");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "rosa_shift_quant: x must be float32, bfloat16 or float16");
  const int64_t rows = B * T;
  if (rows == 0 || d == 0) return KSD_OK;
  if (!x || !sig_q || !sig_k || !sig_v || !q_codes || !q_scales || !k_codes || !k_scales ||
      !v_codes || !v_scales)
    return fail(KSD_EINVAL, "rosa_shift_quant: null pointer");
  const int64_t ng = cdiv(d, group);
  if (rows > 0x7fffffff - 64 || d > (1 << 28) || T > 0x7fffffff)
    return fail(KSD_EINVAL, "rosa_shift_quant: too large");
  const size_t esz = x_dtype == KSD_F32 ? 4 : 2;
  auto al = [](const void *p, size_t a) { return ((uintptr_t)p % a) == 0; };
  const bool vec = d % 8 == 0 && al(x, 16) && (d * esz) % 16 == 0 && al(sig_q, 16) && al(sig_k, 16) &&
                   al(sig_v, 16) && al(q_codes, 8) && al(k_codes, 8) && al(v_codes, 8);
  constexpr int RT = 4;
  const dim3 grid((unsigned)cdiv(rows, 4 * RT), (unsigned)cdiv(d, 512));
  hipStream_t st = (hipStream_t)stream;
#define KSD_SQ(DT, G, V)                                                                         \
  hipLaunchKernelGGL((rosa_shift_quant_kernel<DT, G, V, RT>), grid, dim3(256), 0, st, x, (int)rows,   \
                     (int)T, (int)d, sig_q, sig_k, sig_v, q_codes, q_scales, k_codes, k_scales,   \
                     v_codes, v_scales, (int)ng)
#define KSD_SQ_V(DT, G) \
  if (vec) KSD_SQ(DT, G, true); else KSD_SQ(DT, G, false)
#define KSD_SQ_G(DT) \
  switch (group) { case 32: KSD_SQ_V(DT, 32); break; case 64: KSD_SQ_V(DT, 64); break; default: KSD_SQ_V(DT, 128); }
  switch (x_dtype) {
    case KSD_F32: KSD_SQ_G(KSD_F32); break;
    case KSD_BF16: KSD_SQ_G(KSD_BF16); break;
    default: KSD_SQ_G(KSD_F16); break;
  }
#undef KSD_SQ_G
#undef KSD_SQ_V
#undef KSD_SQ
  return check_launch("rosa_shift_quant");
}

extern "C" int ksd_rosa_shift_quant_dual(const void *x, int x_dtype, int64_t B, int64_t T, int64_t d,
                                         const float *sig_q, const float *sig_k, const float *sig_v,
                                         int8_t *const *codes, uint16_t *const *scales,
                                         int8_t *const *codes_t, uint16_t *const *scales_t,
                                         void *stream) {
  if (B < 0 || T < 0 || d < 0) return fail(KSD_EINVAL, "rosa_shift_quant_dual: negative shape");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "rosa_shift_quant_dual: x must be float32, bfloat16 or float16");
  const int64_t rows = B * T;
  if (rows == 0 || d == 0) return KSD_OK;
  if (!x || !sig_q || !sig_k || !sig_v || !codes || !scales || !codes_t || !scales_t)
    return fail(KSD_EINVAL, "rosa_shift_quant_dual: null pointer");
  ShiftDualOut out;
  for (int m = 0; m < 3; ++m) {
    if (!codes[m] || !scales[m] || !codes_t[m] || !scales_t[m])
      return fail(KSD_EINVAL, "rosa_shift_quant_dual: null output pointer");
    out.codes[m] = codes[m];
    out.scales[m] = scales[m];
    out.codes_t[m] = codes_t[m];
    out.scales_t[m] = scales_t[m];
  }
  if (rows > 0x7fffffff - 256 || d >= (1 << 24))
    return fail(KSD_EINVAL, "rosa_shift_quant_dual: too large");
  const size_t esz = x_dtype == KSD_F32 ? 4 : 2;
  auto al = [](const void *p, size_t a) { return ((uintptr_t)p % a) == 0; };
  bool ok = d % 8 == 0 && al(x, 16) && (d * esz) % 16 == 0 && al(sig_q, 16) && al(sig_k, 16) &&
            al(sig_v, 16);
  for (int m = 0; m < 3; ++m) ok = ok && al(codes[m], 8) && al(scales[m], 2) && al(scales_t[m], 2);
  if (!ok)
    return fail(KSD_EINVAL, "rosa_shift_quant_dual: needs d %% 8 == 0 and 16-byte aligned rows");
  const dim3 grid((unsigned)cdiv(d, 128), (unsigned)cdiv(rows, 128));
  hipStream_t st = (hipStream_t)stream;
  switch (x_dtype) {
    case KSD_F32:
      hipLaunchKernelGGL(rosa_shift_dual_kernel<KSD_F32>, grid, dim3(512), 0, st, x, (int)rows, (int)d,
                         (int)T, sig_q, sig_k, sig_v, out);
      break;
    case KSD_BF16:
      hipLaunchKernelGGL(rosa_shift_dual_kernel<KSD_BF16>, grid, dim3(512), 0, st, x, (int)rows, (int)d,
                         (int)T, sig_q, sig_k, sig_v, out);
      break;
    default:
      hipLaunchKernelGGL(rosa_shift_dual_kernel<KSD_F16>, grid, dim3(512), 0, st, x, (int)rows, (int)d,
                         (int)T, sig_q, sig_k, sig_v, out);
      break;
  }
  return check_launch("rosa_shift_quant_dual");
}

constexpr int kShiftBwdRows = 16;  // rows per wave of rosa_shift_bwd_kernel (4 waves a block)

extern "C" int ksd_rosa_shift_backward_blocks(int64_t B, int64_t T, int64_t *n_blocks) {
  if (!n_blocks || B < 0 || T < 0) return fail(KSD_EINVAL, "rosa_shift_backward_blocks: bad argument");
  *n_blocks = cdiv(B * T, 4 * kShiftBwdRows);
  return KSD_OK;
}

extern "C" int ksd_rosa_shift_backward(const void *x, int x_dtype, int64_t B, int64_t T, int64_t d,
                                       const float *g_q, const float *g_k, const float *g_v,
                                       const float *sig_q, const float *sig_k, const float *sig_v,
                                       void *dx, float *dsig_partials, void *stream) {
  if (B < 0 || T < 0 || d < 0) return fail(KSD_EINVAL, "rosa_shift_backward: negative shape");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "rosa_shift_backward: x must be float32, bfloat16 or float16");
  const int64_t rows = B * T;
  if (rows == 0 || d == 0) return KSD_OK;
  if (!x || !g_q || !g_k || !g_v || !sig_q || !sig_k || !sig_v || !dx || !dsig_partials)
    return fail(KSD_EINVAL, "rosa_shift_backward: null pointer");
  if (rows > 0x7fffffff - 256 || d > (1 << 24)) return fail(KSD_EINVAL, "rosa_shift_backward: too large");
  const size_t esz = x_dtype == KSD_F32 ? 4 : 2;
  auto al = [](const void *p, size_t a) { return ((uintptr_t)p % a) == 0; };
  const bool vec = d % 4 == 0 && al(x, 4 * esz) && al(g_q, 16) && al(g_k, 16) && al(g_v, 16) &&
                   al(sig_q, 16) && al(sig_k, 16) && al(sig_v, 16) && al(dx, 4 * esz);
  const dim3 grid((unsigned)cdiv(d, 256), (unsigned)cdiv(rows, 4 * kShiftBwdRows));
  hipStream_t st = (hipStream_t)stream;
#define KSD_SB(DT, V)                                                                              \
  hipLaunchKernelGGL((rosa_shift_bwd_kernel<DT, kShiftBwdRows, V>), grid, dim3(256), 0, st, x, g_q,  \
                     g_k, g_v, sig_q, sig_k, sig_v, (int)rows, (int)d, (int)T, dx, dsig_partials)
#define KSD_SB_V(DT) \
  if (vec) KSD_SB(DT, true); else KSD_SB(DT, false)
  switch (x_dtype) {
    case KSD_F32: KSD_SB_V(KSD_F32); break;
    case KSD_BF16: KSD_SB_V(KSD_BF16); break;
    default: KSD_SB_V(KSD_F16); break;
  }
#undef KSD_SB_V
#undef KSD_SB
  return check_launch("rosa_shift_backward");
}

static int launch_pack(const PackSrc &ps, int n, int x_dtype, int64_t B, int64_t T, int64_t S,
                       hipStream_t st) {
  const int64_t W = cdiv(T, 32);
  if (W > 65535 || n * B > 65535) return fail(KSD_EINVAL, "rosa_pack_bits: T or B too large");
  dim3 grid((unsigned)cdiv(S, 256), (unsigned)W, (unsigned)(n * B));
  switch (x_dtype) {
    case KSD_F32: hipLaunchKernelGGL(rosa_pack_kernel<KSD_F32>, grid, dim3(256), 0, st, ps, B, T, S, W); break;
    case KSD_BF16: hipLaunchKernelGGL(rosa_pack_kernel<KSD_BF16>, grid, dim3(256), 0, st, ps, B, T, S, W); break;
    default: hipLaunchKernelGGL(rosa_pack_kernel<KSD_F16>, grid, dim3(256), 0, st, ps, B, T, S, W); break;
  }
  return check_launch("rosa_pack_bits");
}

extern "C" int ksd_rosa_pack_bits(const void *x, int x_dtype, int64_t B, int64_t T, int64_t S,
                                  uint32_t *bits, void *stream) {
  if (B < 0 || T < 0 || S < 0) return fail(KSD_EINVAL, "rosa_pack_bits: negative shape");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "rosa_pack_bits: x must be float32, bfloat16 or float16");
  if (B == 0 || T == 0 || S == 0) return KSD_OK;
  if (!x || !bits) return fail(KSD_EINVAL, "rosa_pack_bits: null pointer");
  const PackSrc ps{{x, x, x}, {bits, bits, bits}};
  return launch_pack(ps, 1, x_dtype, B, T, S, (hipStream_t)stream);
}

extern "C" int ksd_rosa_pack_bits3(const void *q, const void *k, const void *v, int x_dtype, int64_t B,
                                   int64_t T, int64_t S, uint32_t *q_bits, uint32_t *k_bits,
                                   uint32_t *v_bits, void *stream) {
  if (B < 0 || T < 0 || S < 0) return fail(KSD_EINVAL, "rosa_pack_bits3: negative shape");
  if (x_dtype != KSD_F32 && x_dtype != KSD_BF16 && x_dtype != KSD_F16)
    return fail(KSD_ETYPE, "rosa_pack_bits3: inputs must be float32, bfloat16 or float16");
  if (B == 0 || T == 0 || S == 0) return KSD_OK;
  if (!q || !k || !v || !q_bits || !k_bits || !v_bits) return fail(KSD_EINVAL, "rosa_pack_bits3: null pointer");
  const PackSrc ps{{q, k, v}, {q_bits, k_bits, v_bits}};
  return launch_pack(ps, 3, x_dtype, B, T, S, (hipStream_t)stream);
}

extern "C" int ksd_rosa_match(const uint32_t *q_bits, const uint32_t *k_bits, const uint32_t *v_bits,
                              int64_t n_streams, int64_t T, int lmax, int8_t *sign, int32_t *match_j,
                              void *stream) {
  if (n_streams < 0 || T < 0) return fail(KSD_EINVAL, "rosa_match: negative shape");
  if (lmax < 0 || lmax > 63) return fail(KSD_EINVAL, "rosa_match: lmax must be in [0, 63]");
  if (T > (1 << 16)) return fail(KSD_EINVAL, "rosa_match: T above 65536 is not supported");
  if (n_streams == 0 || T == 0) return KSD_OK;
  if (!q_bits || !k_bits || !v_bits || !sign) return fail(KSD_EINVAL, "rosa_match: null pointer");
  if (n_streams > 0x7fffffff) return fail(KSD_EINVAL, "rosa_match: too many streams");
  const int W = (int)cdiv(T, 32);
  const int nchunks = (int)cdiv(T, kMatchChunk);
  if (n_streams * nchunks > 0x7fffffffLL) return fail(KSD_EINVAL, "rosa_match: too many streams");
  hipLaunchKernelGGL(rosa_match_kernel, dim3((unsigned)(n_streams * nchunks)), dim3(kMatchChunk),
                     3 * W * sizeof(uint32_t), (hipStream_t)stream, q_bits, k_bits, v_bits, (int)T, W,
                     lmax, (int)n_streams, nchunks, sign, match_j);
  return check_launch("rosa_match");
}

extern "C" int ksd_rosa_hard(const int8_t *sign, const float *payload, int64_t B, int64_t T, int64_t S,
                             void *out, int out_dtype, void *stream) {
  if (B < 0 || T < 0 || S < 0) return fail(KSD_EINVAL, "rosa_hard: negative shape");
  if (out_dtype != KSD_F32 && out_dtype != KSD_BF16 && out_dtype != KSD_F16)
    return fail(KSD_ETYPE, "rosa_hard: out must be float32, bfloat16 or float16");
  if (B == 0 || T == 0 || S == 0) return KSD_OK;
  if (!sign || !payload || !out) return fail(KSD_EINVAL, "rosa_hard: null pointer");
  if (B > 65535 || cdiv(S, 64) > 65535) return fail(KSD_EINVAL, "rosa_hard: B or S too large");
  dim3 grid((unsigned)cdiv(T, 64), (unsigned)cdiv(S, 64), (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
  switch (out_dtype) {
    case KSD_F32: hipLaunchKernelGGL(rosa_hard_kernel<KSD_F32>, grid, dim3(256), 0, st, sign, payload, T, S, out); break;
    case KSD_BF16: hipLaunchKernelGGL(rosa_hard_kernel<KSD_BF16>, grid, dim3(256), 0, st, sign, payload, T, S, out); break;
    default: hipLaunchKernelGGL(rosa_hard_kernel<KSD_F16>, grid, dim3(256), 0, st, sign, payload, T, S, out); break;
  }
  return check_launch("rosa_hard");
}

namespace ksd {

// ---------------------------------------------------------------- exact credits (R5)
// First-order single-bit credits of rosa_credit_gpu.py:28-51 without re-matching per flip.
// For one stream and position t every candidate j < t has a common-suffix length c_j
// (uncapped, <= 64) and cap_j = min(j + 1, lmax); its key is (min(c_j, cap_j), j) and the
// best key decides the sign. Flipping one bit changes candidate lengths in a known way:
//   q[t - i]: c_j < i unchanged; c_j > i -> i; c_j == i -> c_j + 1 + e_j (e_j = the match
//             run after the first mismatch). The new best is the max of the best key with
//             c_j < i (prefix over length buckets), the latest j with c_j > i at length i,
//             and the best extension with c_j == i (per-bucket max).
//   k[p]:     only candidates j in [p, p + lmax) see it, at bit i = j - p: i < c_j truncates
//             to i, i == c_j extends. A truncated key never exceeds the best key, so the sign
//             can change only through (a) an extension beating the best (every candidate
//             that beats it under flip p is such an extension, so the flip's new best is the
//             largest one), or (b) a flip inside the best candidate's matched run: at most
//             lmax flips per t, each resolved from the candidates within 62 of j* (kept in
//             LDS) and the best key farther away (unchanged by the flip).
//   v[p]:     the sign at every t whose endpoint is p - 1 flips (closed form).
// Contributions (sign' - sign) * g(t), g = grad * payload, are added into exact int64
// fixed-point sums (CredAcc below), which a last kernel converts to fp32.


__device__ __forceinline__ int clz64(uint64_t x) { return x ? __clzll((long long)x) : 64; }
// v_ffbh_u32: leading zeros of a word, ~0 for zero
__device__ __forceinline__ uint32_t ffbh32(uint32_t a) {
  uint32_t r;
  asm("v_ffbh_u32 %0, %1" : "=v"(r) : "v"(a));
  return r;
}
// min(a, b, 64) as one v_min3_u32 (kept whole: the compiler would otherwise move the 64
// out of the two branches that compute a lifted length)
__device__ __forceinline__ uint32_t min3_64(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_min3_u32 %0, %1, %2, 64" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ int getbit(const uint32_t *w, int pos) { return (w[pos >> 5] >> (pos & 31)) & 1; }

// key = (length << 16) | (j + 1); length 0 reads as "no match" for the sign.
__device__ __forceinline__ uint32_t mkkey(int len, int j) { return ((uint32_t)len << 16) | (uint32_t)(j + 1); }
__device__ __forceinline__ int key_len(uint32_t k) { return (int)(k >> 16); }
__device__ __forceinline__ int key_j(uint32_t k) { return (int)(k & 0xffffu) - 1; }

__device__ __forceinline__ float sign_of(uint32_t key, const uint32_t *vw) {
  return key_len(key) >= 1 && getbit(vw, key_j(key) + 1) ? 1.0f : -1.0f;
}


// Per-candidate path (scan_position): the 64 lanes of a wave split the candidates j of one
// position t. Per-wave LDS tables for the current t (kScanMw .. words from the base):
//   Mw[65]   best key per common-suffix length c = 0 .. 64
//   Nw[65]   best key per c after flipping the q bit at the first mismatch
//   Rk[128]  k-extension events, slot p mod 128: the best lifted key of flip k[p]
//   tab[256] the near-run flip tables (near_flips_tables)
constexpr int kCredWaves = 4;
constexpr int kScanMw = 0, kScanNw = 72, kScanRk = 144, kScanTab = 272;
constexpr int kCredWave32 = kScanTab + 256;  // uint32 words per wave

// Credit sums. A call runs three kernels: rosa_cred_setup_kernel (per stream: the mode
// below, zeroed sums, d loss / d payload), one of the credit kernels (contributions only,
// into the int64 sums), and rosa_cred_finish_kernel (sums -> fp32 credits). The credits
// buffer is the call's scratch until the last kernel: entries 0 and 1 of every stream hold
// its mode and parameter, entry 3 of the first 64 streams the work counters of the
// balanced kernel.
// Modes, for g = grad * payload over the stream:
//  0  every g finite: every contribution (s' - s) g(t) = +-2 g(t), at most one per position
//     and entry, so with |g| < 2^e an entry stays below 2^(1 + ceil(log2 T) + e). Scaled
//     by 2^k, k = 61 - ceil(log2 T) - e, g(t) is rounded once to an integer (an error below
//     2^-48 of the stream's largest |g|) and the entries are exact int64 sums: the result
//     does not depend on the order in which the atomics land (bit-identical on every run).
//  1  some g = +-inf, none NaN: the reference's dense sum over t of delta * g (rosa_credit_
//     gpu.py:48) makes an entry NaN unless delta != 0 at every infinite position (0 * inf),
//     and then +-inf, or NaN if the infinite terms have both signs; finite terms do not
//     matter. Only the infinite positions are visited, and an entry counts its +inf terms
//     in the high 32 bits and its -inf terms in the low 32 bits.
//  2  some g NaN: every entry is NaN (delta * NaN); nothing is visited.
struct CredAcc {
  unsigned long long *a;  // this stream's (3, T) int64 entries: q at 0, k at T, v at 2T
  double scale;           // 2^k (mode 0)
  bool fin;               // mode 0
  bool scan;              // the stream's positions take the per-candidate path
  // g(t) in fixed point, once per position
  __device__ __forceinline__ long long fixed(float g) const {
    return fin ? (long long)rint((double)g * scale) : 0ll;
  }
  // contribution d * g(t), d = s' - s = +2 (up) or -2
  __device__ __forceinline__ void add(int off, bool up, float g, long long gi) const {
    if (fin) atomicAdd(a + off, (unsigned long long)(up ? 2 * gi : -2 * gi));
    else atomicAdd(a + off, up == (g > 0.0f) ? (1ull << 32) : 1ull);
  }
};

// A stream's mode word in credits entry 0 (a NaN pattern no credit value takes while the
// sums are formed): 0x7fa00000 | idle << 15 | scan << 14 | mode << 12 | (k + 2048) for mode 0,
// where scan selects the per-candidate path for the stream's positions (cred_scan_stream)
// and idle marks a mode-0 stream whose every g is zero (no position to visit).
constexpr uint32_t kCredTag = 0x7fa00000u;
constexpr uint32_t kCredScanBit = 1u << 14, kCredIdleBit = 1u << 15;
__device__ __forceinline__ uint32_t cred_mode_word(int mode, int k, bool scan, bool idle) {
  return kCredTag | (idle ? kCredIdleBit : 0u) | (scan ? kCredScanBit : 0u) | ((uint32_t)mode << 12) |
         (uint32_t)((k + 2048) & 0xfff);
}
// decodes the stream's mode; false when there is nothing to visit (mode 2, or idle)
__device__ __forceinline__ bool cred_acc_of(const float *cred, unsigned long long *sums, int64_t stream,
                                            int T, CredAcc &ca) {
  const uint32_t w = __hip_atomic_load((const uint32_t *)cred + stream * 3 * T, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  const int mode = (int)((w >> 12) & 3u);
  ca.a = sums + stream * 3 * T;
  ca.fin = mode == 0;
  ca.scan = (w & kCredScanBit) != 0u;
  ca.scale = ldexp(1.0, (int)(w & 0xfffu) - 2048);
  return mode != 2 && (w & kCredIdleBit) == 0u;
}
// the positions a mode visits: mode 0 every non-zero g, mode 1 the infinite ones
__device__ __forceinline__ bool cred_live(const CredAcc &ca, float g) {
  return ca.fin ? g != 0.0f : __builtin_isinf(g);
}

constexpr int kCredCounters = 64;  // work counters of the balanced kernel: entry 3 of streams 0, 1, ...

// Path choice of the balanced kernel. The bit-parallel path's cost grows with the size of
// the one-mismatch sets it enumerates, which is large on streams with long runs: many
// positions with a short best match but thousands of one-mismatch candidates, or long
// matches with long extension chains. The per-candidate path costs about the same per
// candidate whatever the stream. Measured per position on random and trained-model
// streams (T 2048), the per-candidate path is the cheaper one when a stream's mean best
// length exceeds 12 or more than 40% of its positions have a best length below 8, and at
// every position below 768 (a scan's cost grows with t, the bit-parallel path's hardly).
constexpr int kScanBelow = 768;
__device__ __forceinline__ bool cred_scan_stream(int64_t len_sum, int64_t short_cnt, int T) {
  return len_sum > 12 * (int64_t)T || 10 * short_cnt > 4 * (int64_t)T;
}

// One block per stream: mode, zeroed sums and d loss / d payload = sum over t of
// grad * sign (rosa_credit_gpu.py:110) in a fixed order: wave w sums t = w, w + 4, ... in
// ascending t, then ((w0 + w1) + w2) + w3. Blocks 0 .. kCredCounters - 1 also zero the work
// counters.
__global__ void __launch_bounds__(256) rosa_cred_setup_kernel(
    const uint32_t *__restrict__ qb, const uint32_t *__restrict__ kb, const uint32_t *__restrict__ vb,
    const int32_t *__restrict__ match_j, const float *__restrict__ grad, const float *__restrict__ payload,
    int64_t S, int T, int W, int lmax, float *__restrict__ cred, float *__restrict__ gp_partial,
    unsigned long long *__restrict__ sums) {
  extern __shared__ uint32_t sm[];
  uint32_t *qw = sm, *kw = sm + W, *vw = sm + 2 * W;
  __shared__ uint32_t red[2 * kCredWaves + 2];
  __shared__ uint32_t lstat[2 * kCredWaves];  // per wave: sum of best lengths, count below 8
  __shared__ float gps[kCredWaves];
  const int64_t stream = blockIdx.x;
  const int64_t b = stream / S, s = stream % S;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < W; i += blockDim.x) {
    qw[i] = qb[stream * W + i];
    kw[i] = kb[stream * W + i];
    vw[i] = vb[stream * W + i];
  }
  __syncthreads();
  const float pay = payload[s];
  float m = 0.0f, gsum = 0.0f;
  int ninf = 0, lsum = 0, lshort = 0;
  bool nan = false;
  for (int t0 = wave; t0 < T; t0 += 64 * kCredWaves) {  // wave-uniform
    const int t = t0 + kCredWaves * lane;
    float gr = 0.0f, term = 0.0f;
    if (t < T) {
      gr = grad[(b * T + t) * S + s];
      const float g = gr * pay;
      if (__builtin_isnan(g)) nan = true;
      else if (__builtin_isinf(g)) ++ninf;
      else m = fmaxf(m, fabsf(g));
      const int jstar = match_j[stream * T + t];
      uint32_t best = 0u;
      if (jstar >= 0) {
        const int cstar = clz64(q_window(qw, t) ^ q_window(kw, jstar));
        best = mkkey(min(cstar, min(jstar + 1, lmax)), jstar);
      }
      term = gr * sign_of(best, vw);
      lsum += key_len(best);
      lshort += key_len(best) < 8;
    }
    // the wave's positions in ascending t: lane order within a chunk of 64
    for (int l = 0; l < 64; ++l) {
      const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, term), l));
      const float gv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gr), l));
      if (gv != 0.0f || gv != gv) gsum += v;  // the credit kernels skip zero gradients
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    m = fmaxf(m, __shfl_xor(m, o));
    ninf += __shfl_xor(ninf, o);
    lsum += __shfl_xor(lsum, o);
    lshort += __shfl_xor(lshort, o);
  }
  const bool wnan = __any(nan);
  if (lane == 0) {
    red[wave] = __builtin_bit_cast(uint32_t, m);
    red[kCredWaves + wave] = (uint32_t)ninf | (wnan ? 0x80000000u : 0u);
    lstat[wave] = (uint32_t)lsum;
    lstat[kCredWaves + wave] = (uint32_t)lshort;
    gps[wave] = gsum;
  }
  __syncthreads();
  float mx = 0.0f;
  uint32_t ni = 0u;
  bool anynan = false;
  int64_t len_sum = 0, short_cnt = 0;
  for (int w = 0; w < kCredWaves; ++w) {
    mx = fmaxf(mx, __builtin_bit_cast(float, red[w]));
    ni += red[kCredWaves + w] & 0x7fffffffu;
    anynan |= (red[kCredWaves + w] >> 31) != 0u;
    len_sum += lstat[w];
    short_cnt += lstat[kCredWaves + w];
  }
  const int mode = anynan ? 2 : (ni ? 1 : 0);
  int k = 0;
  if (mode == 0) {
    int e = 0;
    if (mx > 0.0f) frexpf(mx, &e);  // mx < 2^e
    const int lc = T > 1 ? 32 - __clz(T - 1) : 0;  // ceil(log2 T)
    k = 61 - lc - e;
  }
  unsigned long long *a = sums + stream * 3 * T;
  if (mode != 2)
    for (int i = threadIdx.x; i < 3 * T; i += blockDim.x) a[i] = 0ull;
  if (threadIdx.x == 0) {
    gp_partial[stream] = ((gps[0] + gps[1]) + gps[2]) + gps[3];
    uint32_t *cw = (uint32_t *)cred;
    cw[stream * 3 * T] = cred_mode_word(mode, k, cred_scan_stream(len_sum, short_cnt, (int)T),
                                        mode == 0 && !(mx > 0.0f));
    cw[stream * 3 * T + 1] = ni;
    if (stream < kCredCounters && 3 * T > 3) cw[stream * 3 * T + 3] = 0u;  // a work counter
  }
}

// One block per stream: the sums to fp32 credits. The stream's mode words are entries of
// the output: thread 0 reads them and hands them to the block through LDS before any entry
// is written. (Every wave reading them itself would race with thread 0's first store: the
// compiler may turn such a uniform load into a scalar-cache load placed after the barrier,
// since a 32-bit integer load and the float stores do not alias by type.)
__global__ void __launch_bounds__(256) rosa_cred_finish_kernel(float *cred, const unsigned long long *__restrict__ sums,
                                                               int T) {
  __shared__ uint32_t mw[2];
  const int64_t stream = blockIdx.x;
  uint32_t *f = (uint32_t *)cred + stream * 3 * T;
  const unsigned long long *a = sums + stream * 3 * T;
  if (threadIdx.x == 0) {
    mw[0] = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    mw[1] = __hip_atomic_load(f + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const uint32_t w = mw[0], ninf = mw[1];
  const int mode = (int)((w >> 12) & 3u);
  const double scale = ldexp(1.0, (int)(w & 0xfffu) - 2048);
  const float qnan = __builtin_nanf("");
  for (int i = threadIdx.x; i < 3 * T; i += blockDim.x) {
    float v = qnan;
    if (mode == 0) {
      v = (float)((double)(long long)a[i] / scale);
    } else if (mode == 1) {
      const uint32_t np = (uint32_t)(a[i] >> 32), nn = (uint32_t)a[i];
      if (np + nn == ninf && (np == 0u || nn == 0u)) v = np ? __builtin_inff() : -__builtin_inff();
    }
    f[i] = __builtin_bit_cast(uint32_t, v);
  }
}

__device__ __forceinline__ uint32_t ext_key(int c, int e, int cap, int j) {
  return mkkey(min(c + 1 + e, cap), j);
}

__device__ __forceinline__ void near_flips_tables(int lane, int t, int lmax, int jstar, int trunc_lo,
                                                  int trunc_hi, uint32_t farbest, uint64_t qwin,
                                                  const uint32_t *kw, const uint32_t *vw, float sgn,
                                                  float g, long long gi, const CredAcc &ca, int T,
                                                  uint32_t *tab);
__device__ __forceinline__ uint32_t wave_prefix_max(uint32_t v);

// The per-candidate path for one position t, all lanes of the wave: every candidate's
// common-suffix length from its 64-bit window, 64 candidates per step from the latest down,
// into the bucket tables (Mw: best key per common-suffix bucket, Nw: per bucket after the
// q flip at the first mismatch) and the k-extension events Rk; the flips inside the best
// run from near_flips_tables (tab: 256 words). Writes every table it reads first.
__device__ __forceinline__ void scan_position(int lane, int t, int T, int lmax, uint64_t qwin, uint32_t best,
                                              int jstar, int cstar, int capstar, float sgn, float g,
                                              long long gi, const CredAcc &ca, const uint32_t *kw,
                                              const uint32_t *vw, uint32_t *Mw, uint32_t *Nw, uint32_t *Rk,
                                              uint32_t *tab) {
  const int Lstar = key_len(best);
  // k flips inside the best candidate's matched run, resolved in (b)
  const int trunc_lo = jstar >= 0 ? jstar - min(cstar, capstar) + 1 : 1;
  const int trunc_hi = jstar;
  const int near0 = jstar - 63;  // the near candidates: j in [near0 + 1, near0 + 125]

  Mw[lane] = Nw[lane] = 0u;
  if (lane == 0) Mw[64] = Nw[64] = 0u;
  Rk[lane] = Rk[lane + 64] = 0u;
  uint32_t farbest = 0u;  // best key among j outside [j* - 62, j* + 62] (this lane's j)

  // candidates from the latest down, 64 per step (lane l: j = j0 + l): a bucket's best key is
  // its latest j, so the bucket tables are written only when a key beats the stored one.
  // The step template flags: TOP, the first step (lanes j >= t idle, events above t - 1
  // absent), LOW, the step at j0 = 0 (caps min(j + 1, lmax) below lmax), NEAR: 0 for a step
  // with no candidate in the near range, 1 for one that may have some, 2 to decide at run
  // time. A lane's window words sit at a fixed offset from j0 / 32 and its funnel shift
  // (j + 1) mod 32 is fixed.
  // the lane's window words kw[j0 / 32 + (lane + 1) / 32 - 2 ..], addressed from one LDS
  // address per step (kept opaque, so every step adds one offset to it)
  uint32_t kaddr = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint32_t *)(kw + ((lane + 1) >> 5) - 2);
  asm volatile("" : "+v"(kaddr));
  const int sh = (lane + 1) & 31;
  auto cand_step = [&](int j0, auto top_c, auto low_c, auto near_c) __attribute__((always_inline)) {
    constexpr bool TOP = decltype(top_c)::value, LOW = decltype(low_c)::value;
    constexpr int NEAR = decltype(near_c)::value;
    const int jp1 = (j0 + 1) + lane;  // j + 1, the key's low half
    if (!TOP || jp1 <= t) {
      typedef __attribute__((address_space(3))) const uint32_t lds_u32;
      const uint32_t ka = kaddr + (uint32_t)(j0 >> 5) * 4u;
      const uint32_t wa = *(lds_u32 *)(uintptr_t)ka, wb = *(lds_u32 *)(uintptr_t)(ka + 4u),
                     wc = *(lds_u32 *)(uintptr_t)(ka + 8u);
      const uint64_t kwin = ((uint64_t)__builtin_amdgcn_alignbit(wc, wb, sh) << 32) |
                            __builtin_amdgcn_alignbit(wb, wa, sh);
      const uint64_t x = qwin ^ kwin;
      // c = clz64(x) from the two words: v_ffbh gives ~0 for a zero word, so the low word's
      // count + 32 saturates and the min with 64 covers x = 0
      const uint32_t xh = (uint32_t)(x >> 32);
      const uint32_t lo32 = __builtin_elementwise_add_sat(ffbh32((uint32_t)x), 32u);
      const int c = (int)min(min(ffbh32(xh), lo32), 64u);
      const int cap = LOW ? min(jp1, lmax) : lmax;  // j >= 64 > lmax - 1 above the last step
      const uint32_t key = ((uint32_t)min(c, cap) << 16) | (uint32_t)jp1;
      if (key > Mw[c]) atomicMax(Mw + c, key);
      const bool near_step = NEAR == 2 ? (j0 + 63 > near0 && j0 < near0 + 126) : NEAR == 1;
      if (near_step) {
        if ((unsigned)(jp1 - near0 - 2) > 124u) farbest = max(farbest, key);
      } else {
        farbest = max(farbest, key);
      }
      // the key after flipping the q bit at j's first mismatch (x's top set bit): the
      // common suffix c + 1 + e once that mismatch is gone. With c >= cap the flipped bit
      // lies past the cap and nkey == key; with c = 64 (x = 0, shift taken mod 64) nkey has
      // length 0: it then only reaches Nw[64], which no flip reads.
      // When every lane's first mismatch lies in the window's high word (the common case),
      // the flip leaves the low word as it is, and its leading-zero count is shared with c's.
      int nlen;
      if (__all(c < 32)) {
        nlen = (int)min3_64(ffbh32(xh ^ (0x80000000u >> c)), lo32);
      } else {
        const uint64_t xb = x ^ (0x8000000000000000ull >> (c & 63));
        nlen = (int)min3_64(ffbh32((uint32_t)(xb >> 32)),
                            __builtin_elementwise_add_sat(ffbh32((uint32_t)xb), 32u));
      }
      const uint32_t nkey = ((uint32_t)min(nlen, cap) << 16) | (uint32_t)jp1;
      // (a) flipping k[j - c] extends j past the best (never for c >= cap: nkey == key)
      if (__builtin_expect(nkey > best, 0)) {
        int p = jp1 - c;
        asm volatile("" : "+v"(p));
        p -= 1;
        if (!(p >= trunc_lo && p <= trunc_hi)) atomicMax(Rk + (p & 127), nkey);
      }
      if (nkey > Nw[c]) atomicMax(Nw + c, nkey);
    }
    // events of p come from j in [p, p + 61]: every p >= j0 is now complete (below t)
    {
      const int p = j0 + lane;
      if (!TOP || p < t) {
        uint32_t *slot = Rk + (j0 & 64) + lane;  // slot p mod 128 (j0 is a multiple of 64)
        const uint32_t v = *slot;
        if (v) {
          *slot = 0u;
          const float s2 = sign_of(v, vw);
          // p through an empty asm: the credit address is formed here, not carried as a
          // pointer through every step
          int pe = T + p;
          asm volatile("" : "+v"(pe));
          if (s2 != sgn) ca.add(pe, s2 > 0.0f, g, gi);
        }
      }
    }
  };
  using F_ = std::false_type;
  using T_ = std::true_type;
  using N0 = std::integral_constant<int, 0>;
  using N1 = std::integral_constant<int, 1>;
  using N2 = std::integral_constant<int, 2>;
  const int jtop = ((t - 1) / 64) * 64;
  if (jtop == 0) {
    cand_step(0, T_{}, T_{}, N2{});
  } else {
    cand_step(jtop, T_{}, F_{}, N2{});
    // the middle steps in three runs: above the near range, the (at most three) steps that
    // may reach it, and below it
    int j0 = jtop - 64;
    for (; j0 >= 64 && j0 >= near0 + 126; j0 -= 64) cand_step(j0, F_{}, F_{}, N0{});
    for (; j0 >= 64 && j0 + 63 > near0; j0 -= 64) cand_step(j0, F_{}, F_{}, N1{});
    for (; j0 >= 64; j0 -= 64) cand_step(j0, F_{}, F_{}, N0{});
    cand_step(0, F_{}, T_{}, N2{});
  }
  // (farbest stays per lane: near_flips_tables takes the wave maximum of its own terms)

  // v: the endpoint's successor bit
  if (lane == 0 && Lstar >= 1) ca.add(2 * T + jstar + 1, sgn < 0.0f, g, gi);

  // q: flip of q[t - i], one lane per i in [0, min(L*, lmax - 1)]. Lane c holds bucket c;
  // g1 = max key over buckets < i (exclusive prefix scan), sj = latest j over buckets > i
  // (exclusive suffix scan).
  {
    // DPP prefix maxima; the suffix one over the reversed table, turned back by one shuffle
    // (j + 1 is a key's low half, 0 for an empty bucket)
    // buckets 63 and 64 pooled: a q flip at offset i <= 62 only asks for c < i or c > i
    const uint32_t g1 = wave_prefix_max(lane >= 1 ? Mw[lane - 1] : 0u);  // buckets < lane
    const uint32_t mr = lane == 1 ? max(Mw[63], Mw[64]) : Mw[64 - lane];
    const uint32_t sr = wave_prefix_max(lane >= 1 ? (mr & 0xffffu) : 0u);
    const int sj = (int)(uint32_t)__shfl((int)sr, 63 - lane) - 1;        // buckets > lane
    const int imax = min(min(Lstar, lmax - 1), t);
    if (lane <= imax) {
      const int i = lane;
      uint32_t nb = max(g1, Nw[i]);  // Nw[i]: the candidates with c == i, bit flipped
      if (lane < 63 && sj >= 0) nb = max(nb, mkkey(min(i, min(sj + 1, lmax)), sj));
      const float s2 = sign_of(nb, vw);
      if (s2 != sgn) ca.add(t - i, s2 > 0.0f, g, gi);
    }
  }

  // (b) k flips inside the best candidate's run
  if (jstar >= 0)
    near_flips_tables(lane, t, lmax, jstar, trunc_lo, trunc_hi, farbest, qwin, kw, vw, sgn, g, gi, ca, T, tab);
}

__global__ void __launch_bounds__(256) rosa_credits_kernel(
    const uint32_t *__restrict__ qb, const uint32_t *__restrict__ kb, const uint32_t *__restrict__ vb,
    const int32_t *__restrict__ match_j, const float *__restrict__ grad, const float *__restrict__ payload,
    int64_t S, int T, int W, int lmax, const float *__restrict__ cred,
    unsigned long long *__restrict__ sums) {
  extern __shared__ uint32_t sm[];
  // four zero words before kw: the scan's window loads read kw[-2] and kw[-1] as the
  // positions before 0
  uint32_t *kw = sm + 4, *qw = kw + W, *vw = qw + W;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t *Mw = sm + 4 + 3 * W + wave * kCredWave32 + kScanMw;
  uint32_t *Nw = Mw + kScanNw, *Rk = Mw + kScanRk;
  uint32_t *tab = Mw + kScanTab;
  const int64_t stream = blockIdx.x;
  const int64_t b = stream / S, s = stream % S;
  if (threadIdx.x < 4) sm[threadIdx.x] = 0u;
  for (int i = threadIdx.x; i < W; i += 256) {
    qw[i] = qb[stream * W + i];
    kw[i] = kb[stream * W + i];
    vw[i] = vb[stream * W + i];
  }
  __syncthreads();
  const float pay = payload[s];
  CredAcc ca;
  if (!cred_acc_of(cred, sums, stream, T, ca)) return;  // block-uniform

  for (int t = wave; t < T; t += kCredWaves) {  // wave-uniform
    const float gr = grad[(b * T + t) * S + s];
    const int jstar = match_j[stream * T + t];
    const uint64_t qwin = q_window(qw, t);
    uint32_t best = 0u;
    int cstar = 0, capstar = 0;
    if (jstar >= 0) {
      cstar = clz64(qwin ^ q_window(kw, jstar));
      capstar = min(jstar + 1, lmax);
      best = mkkey(min(cstar, capstar), jstar);
    }
    const float sgn = sign_of(best, vw);
    const float g = gr * pay;
    if (t == 0 || !cred_live(ca, g) || lmax < 1) continue;
    const long long gi = ca.fixed(g);
    scan_position(lane, t, T, lmax, qwin, best, jstar, cstar, capstar, sgn, g, gi, ca, kw, vw, Mw, Nw, Rk, tab);
  }
}

// Bit-parallel credits for streams of up to 2048 positions (W <= 64 words). Same outputs as
// rosa_credits_kernel. For position t, lane w of a wave holds word w of every candidate
// set (bit b = candidate j = 32 w + b, j < t), and the levels L of the common-suffix chain
// are processed a whole set at a time:
//   D_L  = {j >= L : k[j - L] == q[t - L]}      (one alignbit of the lane's k words)
//   A_L  = {j : the first L positions match}     A_0 = [0, t),  A_{L+1} = A_L & D_L
//   O_L  = {j : exactly one mismatch in the first L positions, j >= L - 1}
//          O_{L+1} = (O_L & D_L) | (A_L & ~D_L & {j >= L})
// A_L holds the candidates whose key length (capped by min(j + 1, lmax)) is at least L.
// O_L holds those whose "lifted" length is at least L: with the bit of their single
// mismatch flipped they would match L positions.
//  q flip at offset i (i <= min(L*, lmax - 1)): the new best is the longest lifted member
//    of bucket i (the candidates whose first mismatch is at i), if the bucket has one
//    within its cap; otherwise (i, latest j of A_i). The bucket maxima come from the
//    members of O at the checkpoint levels L*, L* - 3 and L* - 6: a member with lifted
//    length >= L lies in O_L. Each member gets its first mismatch c and lifted length from
//    its 64-bit window. A bucket no checkpoint covers is resolved by its own chain.
//  k flip at p outside the best run: the largest lifted key among the members j of
//    O_{L*+1} u (O_{L*} & {j > j*}) with j - c_j = p (a per-p table), if any.
//  k flip inside the best run, and v flips: as in rosa_credits_kernel.
// LDS per wave: one 64-word bucket table (the best lifted key of a bucket with members,
// the latest j of A_i for one without: the two never meet in a bucket), the work item's
// q/k/v words, and the per-p event table in 16-bit entries, two to a word. For one p the
// members' keys order as their (lifted length, c) pairs do (j = p + c), so an entry holds
// (length << 6) | c, at most 12 bits. The near-run flip tables (256 words) reuse the event
// table's first words: the k-flip pass leaves every event entry zero before they are
// written, and they are cleared after use. 5 KB per wave lets 8 four-wave blocks share a
// CU. Every wave works alone (no block barrier): the block is only a unit of launch.
constexpr int kBpMaxT = 2048;
constexpr int kCredChunk = 16;        // positions per work item
constexpr int kBpWave32 = 64 + 3 * 64 + kBpMaxT / 2;  // u32 words per wave
constexpr int kBpBlocksPerCu = 8;
// the per-candidate path's tables and their clearing stay below the event table's last
// two words, which the k words' window loads read as zero
static_assert(64 * ((kCredWave32 + 63) / 64) <= kBpMaxT / 2 - 2, "scan tables overlap kw[-2..-1]");     // 20 KB of LDS per block: 8 blocks fill a CU's 160 KB

__device__ __forceinline__ uint32_t evt_key16(uint32_t key, int c) {
  return ((uint32_t)key_len(key) << 6) | (uint32_t)c;
}
// entry p := max(entry p, k16); the word's other entry may be updated by another lane at
// the same time, hence the compare-and-swap
// The table lives in LDS; the volatile accesses go through LDS-typed pointers (the low 32
// bits of a generic pointer into LDS are its LDS offset), so they compile to ds_* and not
// to flat accesses.
typedef __attribute__((address_space(3))) volatile uint32_t lds_vu32;
typedef __attribute__((address_space(3))) volatile uint16_t lds_vu16;
__device__ __forceinline__ void evt_max16(uint32_t *evt, int p, uint32_t k16) {
  uint32_t *w = evt + (p >> 1);
  const int sh = (p & 1) * 16;
  uint32_t old = *(lds_vu32 *)(uint32_t)(uintptr_t)w;
  while (((old >> sh) & 0xffffu) < k16) {
    const uint32_t prev = atomicCAS(w, old, (old & ~(0xffffu << sh)) | (k16 << sh));
    if (prev == old) break;
    old = prev;
  }
}
__device__ __forceinline__ uint32_t evt_get16(const uint32_t *evt, int p) {
  return ((lds_vu16 *)(uint32_t)(uintptr_t)evt)[p];
}
__device__ __forceinline__ void evt_clear16(uint32_t *evt, int p) {
  ((lds_vu16 *)(uint32_t)(uintptr_t)evt)[p] = 0;
}

__device__ __forceinline__ int set_maxbit(uint32_t word) {  // highest candidate of a wave set
  const uint64_t bal = __ballot(word != 0u);
  if (bal == 0) return -1;
  const int hl = 63 - __clzll((long long)bal);
  const uint32_t hw = (uint32_t)__builtin_amdgcn_readlane((int)word, hl);  // hl is wave-uniform
  return 32 * hl + 31 - __clz(hw);
}

// Inclusive prefix max over the wave's 64 lanes by DPP (all lanes active): shifts by 1, 2,
// 4 and 8 within each row of 16, then the last lane of rows 0 and 2 into rows 1 and 3
// (row_bcast:15), then lane 31 into rows 2 and 3 (row_bcast:31). A lane without a source
// reads 0, the identity of the max over unsigned keys.
__device__ __forceinline__ uint32_t wave_prefix_max(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));
  return v;
}

// k flips inside the best run p in [trunc_lo, trunc_hi] (one lane per p, i = p - trunc_lo
// < 62), from the near candidates j in [j* - 62, j* + 62] (two per lane). With a near
// candidate's unchanged key K = (m, j), m = min(c, cap), a flip at p
//   leaves K unchanged when p > j, or when p < s = j - m (+1 if the mismatch at j - m is
//     the cap, which a flip there does not lift),
//   truncates it to (j - p, j) when j - m < p <= j,
//   lifts it to its extended key when p = j - c < j - m + 1, i.e. c < cap.
// So the new best is the max of: the far best (farbest, no far key changes), the near keys
// with j < p (prefix max), those with s > p (suffix max over s), the truncation (j_t - p,
// j_t) with j_t the latest j >= j* whose run covers p (prefix max of j over run starts;
// earlier j give smaller keys than j* itself), and the lifted keys with j - c = p. Each
// term is a 64-entry table indexed by i, filled by scatter and scanned across the wave.
__device__ __forceinline__ void near_flips_tables(int lane, int t, int lmax, int jstar, int trunc_lo,
                                                  int trunc_hi, uint32_t farbest, uint64_t qwin,
                                                  const uint32_t *kw, const uint32_t *vw, float sgn,
                                                  float g, long long gi, const CredAcc &ca, int T,
                                                  uint32_t *tab) {
  uint32_t *PK = tab, *SU = tab + 64, *TJ = tab + 128, *LF = tab + 192;
  PK[lane] = 0u;  // PK[j - trunc_lo]: the key of j in the run
  SU[lane] = 0u;
  TJ[lane] = 0u;
  LF[lane] = 0u;
  __builtin_amdgcn_wave_barrier();
  const int jlo = max(0, jstar - 62), jhi = min(t - 1, jstar + 62);
  uint32_t always = farbest;  // keys no flip of the run changes: far, j < trunc_lo, s > trunc_hi + 1
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int j2 = jstar - 63 + 2 * lane + h;
    if (j2 >= jlo && j2 <= jhi) {
      const uint64_t x2 = qwin ^ q_window(kw, j2);
      const int c2 = clz64(x2);
      const int cap2 = min(j2 + 1, lmax);
      const int m2 = min(c2, cap2);
      const uint32_t key = mkkey(m2, j2);
      const bool lift = c2 < cap2;
      const int su = lift ? j2 - m2 : j2 - m2 + 1;
      if (j2 < trunc_lo || su > trunc_hi + 1) always = max(always, key);
      else if (su > trunc_lo) atomicMax(SU + su - trunc_lo, key);
      if (j2 >= trunc_lo && j2 <= trunc_hi) PK[j2 - trunc_lo] = key;
      const int sr = j2 - m2 + 1;
      if (j2 >= jstar && sr <= trunc_hi) atomicMax(TJ + max(sr, trunc_lo) - trunc_lo, (uint32_t)(j2 + 1));
      const int pl = j2 - c2;
      if (lift && pl >= trunc_lo && pl <= trunc_hi)
        atomicMax(LF + pl - trunc_lo, ext_key(c2, clz64(x2 << (c2 + 1)), cap2, j2));
    }
  }
  // wave max of `always`: rows of 16 by DPP, then the four row results
  always = group_max_u32<16>(always);
  always = max(max((uint32_t)__builtin_amdgcn_readlane((int)always, 0), (uint32_t)__builtin_amdgcn_readlane((int)always, 16)),
               max((uint32_t)__builtin_amdgcn_readlane((int)always, 32), (uint32_t)__builtin_amdgcn_readlane((int)always, 48)));
  __builtin_amdgcn_wave_barrier();
  // prefix max of PK (j < p: entries .. i - 1) and TJ; the suffix max of SU (s > p:
  // entries i + 1 ..) as a prefix max over the reversed table, turned back by one shuffle
  const uint32_t pk = wave_prefix_max(lane >= 1 ? PK[lane - 1] : 0u);
  const uint32_t tj = wave_prefix_max(TJ[lane]);
  const uint32_t sr = wave_prefix_max(lane >= 1 ? SU[64 - lane] : 0u);
  const uint32_t su = (uint32_t)__shfl((int)sr, 63 - lane);
  const uint32_t lf = LF[lane];
  const int p = trunc_lo + lane;
  if (p <= trunc_hi) {
    const int jt = (int)tj - 1;  // >= j*: j* covers every p of its run
    uint32_t nb = max(max(always, pk), max(su, lf));
    nb = max(nb, mkkey(jt - p, jt));
    const float s2 = sign_of(nb, vw);
    if (s2 != sgn) ca.add(T + p, s2 > 0.0f, g, gi);
  }
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) rosa_credits_bp_kernel(
    const uint32_t *__restrict__ qb, const uint32_t *__restrict__ kb, const uint32_t *__restrict__ vb,
    const int32_t *__restrict__ match_j, const float *__restrict__ grad, const float *__restrict__ payload,
    int64_t S, int T, int W, int lmax, const float *__restrict__ cred, unsigned long long *__restrict__ sums,
    unsigned int *__restrict__ counters, int64_t cstride, int ncount, int nstreams, int nchunks, int force) {
  __shared__ __attribute__((aligned(16))) uint32_t wsm[kCredWaves][kBpWave32];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // [64] per bucket i: the best lifted key when the bucket has members (hasext bit i),
  // else the latest j of A_i; the two never meet in one bucket
  // per wave: Nw [64], the item's q and v words [64 each], evt, the item's k words [64]
  // (after evt, whose last words are zero whenever the per-candidate path runs: the scan's
  // window loads read kw[-2] and kw[-1] as the positions before 0)
  uint32_t *Nw = wsm[wave];
  uint32_t *qw = Nw + 64, *vw = qw + 64;
  uint32_t *evt = Nw + 192;                       // [kBpMaxT] 16-bit event entries per flip p
  uint32_t *kw = evt + kBpMaxT / 2;
  uint32_t *ntab = evt;                           // [256] near-flip tables (aliasing evt)
  for (int i = lane; i < 64; i += 64) Nw[i] = 0u;
  for (int i = lane; i < kBpMaxT / 2; i += 64) evt[i] = 0u;
  // {j >= L} for this lane's word as the low 32 bits of p01 >> (32 - L) (L <= 32) or
  // p12 >> (64 - L) (L > 32): only words 0 and 1 hold positions below 63
  const uint64_t p01 = lane == 0 ? ~0ull << 32 : ~0ull;
  const uint64_t p12 = lane == 0 ? 0ull : (lane == 1 ? ~0ull << 32 : ~0ull);
  const int nitems = nstreams * nchunks;
  // Work items (stream, chunk of kCredChunk positions): the cost of a position grows with t
  // and varies widely between streams (long matches cost far more), so the waves take
  // items dynamically, the later chunks of every stream first, until none is left. Item i
  // belongs to counter i % ncount (the counters sit ncount apart: one counter for all
  // items would serialize every wave's fetch on one address); a wave starts at its own
  // counter and moves to the next one once that is spent, reading a counter before adding
  // to it so that spent ones cost no atomic.
  const int wid = (int)blockIdx.x * kCredWaves + wave;
  int cc = wid % ncount, spent = 0;
  for (;;) {
    const int lim = (nitems - cc + ncount - 1) / ncount;  // local indices of counter cc
    int item = nitems;
    if (__hip_atomic_load(counters + cc * cstride, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT) < (unsigned int)lim) {
      unsigned int it = 0u;
      if (lane == 0) it = atomicAdd(counters + cc * cstride, 1u);
      const int l = __builtin_amdgcn_readfirstlane((int)it);
      if (l < lim) item = cc + l * ncount;
    }
    if (item >= nitems) {  // wave-uniform: counter cc is spent
      if (++spent == ncount) break;
      cc = cc + 1 == ncount ? 0 : cc + 1;
      continue;
    }
    const int chunk = nchunks - 1 - item / nstreams;
    const int64_t stream = item % nstreams;
    CredAcc ca;
    if (!cred_acc_of(cred, sums, stream, T, ca)) continue;  // nothing to visit in the stream
    const int64_t b = stream / S, s = stream % S;
    // the chunk's positions: the lanes load their gradients and endpoints together, and only
    // the positions the stream's mode visits are walked (an item without one loads no words)
    const float pay = payload[s];
    const int tl = chunk * kCredChunk + lane;
    const float grl = lane < kCredChunk && tl < T ? grad[(b * T + tl) * S + s] : 0.0f;
    uint64_t live = __ballot(lane < kCredChunk && tl < T && cred_live(ca, grl * pay));
    if (!live) continue;
    const int mjl = lane < kCredChunk && tl < T ? match_j[stream * T + tl] : -1;
    __builtin_amdgcn_wave_barrier();
    qw[lane] = lane < W ? qb[stream * W + lane] : 0u;
    kw[lane] = lane < W ? kb[stream * W + lane] : 0u;
    vw[lane] = lane < W ? vb[stream * W + lane] : 0u;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // this lane's k words: word w and the two below it (zeros before position 0)
    const uint32_t k0 = kw[lane], k1 = lane >= 1 ? kw[lane - 1] : 0u, k2 = lane >= 2 ? kw[lane - 2] : 0u;
    const uint64_t k01 = ((uint64_t)k0 << 32) | k1, k12 = ((uint64_t)k1 << 32) | k2;
    // every position's prologue at once, lane l for position chunk * kCredChunk + l: its q
    // window, the best key from the endpoint, the current sign and g in fixed point
    uint64_t qwl = 0;
    uint32_t bestl = 0u;
    int cstarl = 0;
    long long gil = 0;
    if (lane < kCredChunk && tl < T) {
      qwl = q_window(qw, tl);
      if (mjl >= 0) {
        cstarl = clz64(qwl ^ q_window(kw, mjl));
        bestl = mkkey(min(cstarl, min(mjl + 1, lmax)), mjl);
      }
      gil = ca.fixed(grl * pay);
    }
    const float sgnl = sign_of(bestl, vw);
    while (live) {  // wave-uniform
    const int li = __builtin_ctzll(live);
    live &= live - 1;
    const int t = chunk * kCredChunk + li;
    if (t == 0 || lmax < 1) continue;
    const float gr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, grl), li));
    const int jstar = __builtin_amdgcn_readlane(mjl, li);
    const uint64_t qwin = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(qwl >> 32), li) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)qwl, li);
    const uint32_t best = (uint32_t)__builtin_amdgcn_readlane((int)bestl, li);
    const int cstar = __builtin_amdgcn_readlane(cstarl, li);
    const int capstar = jstar >= 0 ? min(jstar + 1, lmax) : 0;
    const float sgn = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sgnl), li));
    const float g = gr * pay;
    const long long gi = (long long)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(gil >> 32), li) << 32) |
                                     (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)gil, li));
    if (force == 2 || (force == 0 && (ca.scan || t < kScanBelow))) {  // wave-uniform
      // the per-candidate path, its tables in the event table's first kCredWave32 words
      scan_position(lane, t, T, lmax, qwin, best, jstar, cstar, capstar, sgn, g, gi, ca, kw, vw,
                    evt + kScanMw, evt + kScanNw, evt + kScanRk, evt + kScanTab);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < (kCredWave32 + 63) / 64; ++i) evt[64 * i + lane] = 0u;  // the bit-parallel path expects zeros
      __builtin_amdgcn_wave_barrier();
      continue;
    }
    const int Ls = key_len(best);
    if (lane == 0 && Ls >= 1) ca.add(2 * T + jstar + 1, sgn < 0.0f, g, gi);  // v flips
    const int imax = min(min(Ls, lmax - 1), t);
    const int trunc_lo = jstar >= 0 ? jstar - min(cstar, capstar) + 1 : 1;
    const int trunc_hi = jstar;

    // masks of this lane's word: candidates j < t, and j outside [j* - 62, j* + 62]
    const int tw = t >> 5;
    const uint32_t valid = lane < tw ? ~0u : (lane == tw ? (1u << (t & 31)) - 1u : 0u);
    uint32_t farm = ~0u;
    if (jstar >= 0) {
      const int lo = jstar - 62, hi = jstar + 62, w0b = 32 * lane;  // near range [lo, hi]
      const int a = max(lo - w0b, 0), e = min(hi - w0b, 31);        // its bits in this word
      if (a <= e) farm = ~(((e - a == 31) ? ~0u : ((2u << (e - a)) - 1u)) << a);
    }
    // D_L and its complement {j >= L : mismatch at L} for this lane, without branches
    // (L is wave-uniform): k[j - L] for the word's 32 j is one funnel shift of the word
    // pair (k0:k1) for L <= 32 or (k1:k2) above, and {j >= L} the same shift of a per-lane
    // constant pair (HI picks the pair at compile time where the level range is known)
    auto level_c = [&](auto hi_c, int L, uint32_t &D, uint32_t &Dn) __attribute__((always_inline)) {
      constexpr bool HI = decltype(hi_c)::value;
      const int sh = (HI ? 64 : 32) - L;
      const uint32_t KL = (uint32_t)((HI ? k12 : k01) >> sh);
      const uint32_t pos = (uint32_t)((HI ? p12 : p01) >> sh);
      const uint32_t qm = 0u - (uint32_t)((qwin >> (63 - L)) & 1ull);  // q[t - L] ? ~0 : 0
      D = (KL ^ ~qm) & pos;
      Dn = pos & ~D;
    };
    auto level = [&](int L, uint32_t &D, uint32_t &Dn) __attribute__((always_inline)) {
      if (L > 32) level_c(std::true_type{}, L, D, Dn);
      else level_c(std::false_type{}, L, D, Dn);
    };

    // ascending pass over the levels 0 .. min(lmax, L* + 1) - 1: the levels below
    // L* - 7 only advance A, O and the extension flags; the last eight (unrolled) also
    // record the checkpoints O_{L*-6}, O_{L*-3}, O_{L*}, O_{L*+1}, the latest j of A_L
    // for L >= L* - 2, and the far candidates
    uint32_t A = valid, O = 0u, O6 = 0u, O3 = 0u, Os = 0u, Os1 = 0u;
    uint64_t hasext = 0;
    uint32_t farw = 0u;
    int farL = -1;
    const int Lend = min(lmax, Ls + 1);
    const int L0 = min(max(0, Ls - 7), Lend);
    auto step = [&](auto hi_c, int L, bool tail) __attribute__((always_inline)) {
      uint32_t D, Dn;
      level_c(hi_c, L, D, Dn);
      if (L <= imax) {
        if (__any((A & Dn) != 0u)) {
          hasext |= 1ull << L;
        } else if (L >= 1) {  // a q flip at offset L without an extension: latest j of A_L
          const int lj = set_maxbit(A);
          if (lane == 0) Nw[L] = (uint32_t)lj;
        }
      }
      if (tail) {
        if (__any((A & farm) != 0u)) {
          farw = A & farm;
          farL = L;
        }
      }
      O = (O & D) | (A & Dn);
      A &= D;
    };
    int Lm = 0;
    for (; Lm < min(L0, 33); ++Lm) step(std::false_type{}, Lm, false);
    for (; Lm < L0; ++Lm) step(std::true_type{}, Lm, false);
    const bool far_below = L0 > 0 && !__any((A & farm) != 0u);  // far best below the tail
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      const int Lt = Ls - 7 + s8;
      if (Lt >= 0 && Lt < Lend) {  // wave-uniform
        if (Lt > 32) step(std::true_type{}, Lt, true);
        else step(std::false_type{}, Lt, true);
        if (s8 == 0) O6 = O;
        if (s8 == 3) O3 = O;
        if (s8 == 6) Os = O;
        if (s8 == 7) Os1 = O;
      }
    }
    if (Lend == Ls && __any((A & farm) != 0u)) {  // L* = lmax: A_{L*} is still non-empty
      farw = A & farm;
      farL = Lend;
    }
    if (far_below && __any((valid & farm) != 0u)) {  // the far candidates' own chain:
      uint32_t Af = valid & farm, D, Dn;               // the last level where any survives
      int L = 0;
      for (; L < L0; ++L) {
        level(L, D, Dn);
        if (!__any((Af & D) != 0u)) break;
        Af &= D;
      }
      farw = Af;
      farL = L;
    }

    // members of a checkpoint set: bucket maxima, and (ev) the lifted keys per flip p
    // The event updates of one lane are merged while its consecutive members name the same
    // flip p, and a wave whose last pending updates all name one p sends one update: in a
    // long run every member's first mismatch is the same k bit, and evt_max16's
    // compare-and-swap serializes the lanes that update one entry.
    auto members = [&](uint32_t x, bool ev) __attribute__((always_inline)) {
      int pp = -1;       // this lane's pending event: flip p and its max entry
      uint32_t pk = 0u;
      while (__any(x != 0u)) {
        if (x != 0u) {
          const int bb = 31 - __clz(x);
          x &= ~(1u << bb);
          const int j = 32 * lane + bb;
          const uint64_t hi = ((uint64_t)k0 << 32) | k1;
          const uint64_t kwin = (hi << (31 - bb)) | (bb == 31 ? 0ull : ((uint64_t)k2 >> (bb + 1)));
          const uint64_t xx = qwin ^ kwin;
          const int c = clz64(xx);               // < cap for every member of O
          const int e = clz64(xx << (c + 1));
          const uint32_t key = ext_key(c, e, min(j + 1, lmax), j);
          if (c <= imax) atomicMax(Nw + c, key);
          const int p = j - c;
          if (ev && key > best && !(p >= trunc_lo && p <= trunc_hi)) {
            const uint32_t k16 = evt_key16(key, c);
            if (p == pp) {
              pk = max(pk, k16);
            } else {
              if (pp >= 0) evt_max16(evt, pp, pk);
              pp = p;
              pk = k16;
            }
          }
        }
      }
      const uint64_t pend = __ballot(pp >= 0);
      if (pend) {  // wave-uniform
        const int lead = __builtin_ctzll(pend);
        const int p0 = __builtin_amdgcn_readlane(pp, lead);
        if (__all(pp < 0 || pp == p0)) {
          uint32_t m = pp >= 0 ? pk : 0u;
#pragma unroll
          for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o));
          if (lane == lead) evt_max16(evt, p0, m);
        } else if (pp >= 0) {
          evt_max16(evt, pp, pk);
        }
      }
    };
    auto unresolved = [&]() __attribute__((always_inline)) -> uint64_t {
      return __ballot(lane <= imax && ((hasext >> lane) & 1ull) && Nw[lane] == 0u);
    };
    // candidates that mismatch at one of the offsets i < lc of the buckets u: a member of
    // a checkpoint set O_lc has one mismatch, at its bucket c < lc, so this mask keeps
    // every member of those buckets (members of other buckets only repeat a max)
    auto bucket_mask = [&](uint64_t u, int lc) __attribute__((always_inline)) -> uint32_t {
      u &= (1ull << lc) - 1ull;  // 1 <= lc <= 62
      uint32_t msk = 0u;
      while (u) {
        const int i = __ffsll((long long)u) - 1;
        u &= u - 1;
        uint32_t D, Dn;
        level(i, D, Dn);
        msk |= Dn;
      }
      return msk;
    };
    members(Os | Os1, true);
    uint64_t U = unresolved();
    if (U && Ls - 3 >= 1) {
      members(O3 & ~Os & bucket_mask(U, Ls - 3), false);
      U = unresolved();
      if (U && Ls - 6 >= 1) {
        members(O6 & ~O3 & bucket_mask(U, Ls - 6), false);
        U = unresolved();
      }
    }
    // U: buckets with every lifted length below the last checkpoint need A_i again: their
    // candidates A_i & Dn_i are extended level by level until none survives, walked in
    // ascending i along one chain
    {
      uint64_t W = U;
      uint32_t Ach = valid;  // A_Lch
      int Lch = 0;
      while (W) {
        const int i = __ffsll((long long)W) - 1;
        W &= W - 1;
        uint32_t D, Dn;
        for (; Lch < i; ++Lch) {
          level(Lch, D, Dn);
          Ach &= D;
        }
        level(i, D, Dn);
        uint32_t Tt = Ach & Dn;
        int L = i + 1;
        for (; L < lmax; ++L) {
          level(L, D, Dn);
          const uint32_t T2 = Tt & D;
          if (!__any(T2 != 0u)) break;
          Tt = T2;
        }
        const int jp = set_maxbit(Tt);
        if (lane == 0) Nw[i] = mkkey(L, jp);
      }
    }

    // q flips: one lane per offset i
    if (lane <= imax) {
      const int i = lane;
      const uint32_t nb = ((hasext >> i) & 1ull) ? Nw[i] : (i >= 1 ? mkkey(i, (int)Nw[i]) : 0u);
      const float s2 = sign_of(nb, vw);
      if (s2 != sgn) ca.add(t - i, s2 > 0.0f, g, gi);
    }
    Nw[lane] = 0u;

    // k flips outside the best run: every event member checks whether it holds its flip's
    // maximum; the holder adds the contribution and clears the entry
    {
      uint32_t x = Os1;
      if (Ls >= 1) {
        const int jb = jstar + 1 - 32 * lane;  // bits j > j* in this word
        x |= Os & (jb <= 0 ? ~0u : (jb >= 32 ? 0u : ~0u << jb));
      }
      while (__any(x != 0u)) {
        if (x != 0u) {
          const int bb = 31 - __clz(x);
          x &= ~(1u << bb);
          const int j = 32 * lane + bb;
          const uint64_t hi = ((uint64_t)k0 << 32) | k1;
          const uint64_t kwin = (hi << (31 - bb)) | (bb == 31 ? 0ull : ((uint64_t)k2 >> (bb + 1)));
          const uint64_t xx = qwin ^ kwin;
          const int c = clz64(xx);
          const int e = clz64(xx << (c + 1));
          const uint32_t key = ext_key(c, e, min(j + 1, lmax), j);
          const int p = j - c;
          if (!(p >= trunc_lo && p <= trunc_hi) && evt_get16(evt, p) == evt_key16(key, c)) {
            evt_clear16(evt, p);
            const float s2 = sign_of(key, vw);
            if (s2 != sgn) ca.add(T + p, s2 > 0.0f, g, gi);
          }
        }
      }
    }

    // k flips inside the best run, from the candidates near j*
    if (jstar >= 0) {
      const uint32_t farbest = farL >= 0 ? mkkey(farL, set_maxbit(farw)) : 0u;
      near_flips_tables(lane, t, lmax, jstar, trunc_lo, trunc_hi, farbest, qwin, kw, vw, sgn, g, gi, ca, T, ntab);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int k = 0; k < 4; ++k) ntab[64 * k + lane] = 0u;  // the event entries they covered
      __builtin_amdgcn_wave_barrier();
    }
    }
  }
}

// d loss / d payload = sum over (b, t) of grad * sign (rosa_credit_gpu.py:110), and the
// Bernoulli map of the credits to projection space (:99-111),
//   g = (credit (1 - 2 bit))_DT * (sigmoid(x) (1 - sigmoid(x)))_DT,  bit = x > 0,
// each factor rounded to x's dtype as the reference's tensor ops are. The credits are laid
// out (b, s, m, t) and the projections (b, t, s): a block takes a 64 (t) x 64 (s) tile,
// reads the three credit tiles along t into LDS (pitch 65) and writes along s.
constexpr int kCgTile = 64;

template <int DT>
__global__ void __launch_bounds__(256) rosa_credit_grad_kernel(
    const float *__restrict__ cred, const void *__restrict__ q, const void *__restrict__ k,
    const void *__restrict__ v, int64_t B, int64_t T, int64_t S, void *__restrict__ gq,
    void *__restrict__ gk, void *__restrict__ gv) {
  using E = Elem<DT>;
  __shared__ float tile[3][kCgTile][kCgTile + 1];  // [m][s][t]
  const int64_t s0 = (int64_t)blockIdx.x * kCgTile, t0 = (int64_t)blockIdx.y * kCgTile, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // load: wave w takes streams s0 + w, w + 4, ...; a lane one position t0 + lane
  for (int sl = wave; sl < kCgTile; sl += 4) {
    const int64_t s = s0 + sl, t = t0 + lane;
    const bool ok = s < S && t < T;
    const float *c = cred + (b * S + (ok ? s : 0)) * 3 * T + (ok ? t : 0);
#pragma unroll
    for (int m = 0; m < 3; ++m) tile[m][sl][lane] = ok ? c[m * T] : 0.0f;
  }
  __syncthreads();
  const void *pre[3] = {q, k, v};
  void *out[3] = {gq, gk, gv};
  // compute: a lane takes stream s0 + lane, wave w positions t0 + w, w + 4, ...
  const int64_t s = s0 + lane;
  if (s >= S) return;  // after the block's only barrier
  for (int tl = wave; tl < kCgTile; tl += 4) {
    const int64_t t = t0 + tl;
    if (t >= T) break;
    const int64_t idx = (b * T + t) * S + s;
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      const float x = E::load((const typename E::T *)pre[m] + idx);
      const float bit = x > 0.0f ? 1.0f : 0.0f;
      const float delta = round_to_dt<DT>(tile[m][lane][tl] * (1.0f - 2.0f * bit));
      const float sg = 1.0f / (1.0f + expf(-x));
      const float bern = round_to_dt<DT>(sg * (1.0f - sg));
      store_out<DT>(out[m], idx, delta * bern);
    }
  }
}

// d payload[s] = sum over b of the per-stream partials, in a fixed order.
__global__ void __launch_bounds__(256) rosa_payload_grad_kernel(const float *__restrict__ partial,
                                                                int64_t B, int64_t S,
                                                                float *__restrict__ gp) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= S) return;
  float acc = 0.0f;
  for (int64_t b = 0; b < B; ++b) acc += partial[b * S + s];
  gp[s] = acc;
}

}  // namespace ksd

using namespace ksd;

// KSD_ROSA_CREDITS_PATH = "bits" or "scan" makes every position of the balanced kernel take
// one path (both give identical sums; for tests and measurement); unset or anything else
// lets each stream's statistics and the position choose.
static int credits_path_override() {
  const char *e = getenv("KSD_ROSA_CREDITS_PATH");
  if (e && !strcmp(e, "bits")) return 1;
  if (e && !strcmp(e, "scan")) return 2;
  return 0;
}

extern "C" int ksd_rosa_credits(const uint32_t *q_bits, const uint32_t *k_bits, const uint32_t *v_bits,
                                const int32_t *match_j, const float *grad, const float *payload,
                                int64_t B, int64_t T, int64_t S, int lmax, float *credits,
                                float *payload_partial, int64_t *credit_sums, void *stream) {
  if (B < 0 || T < 0 || S < 0) return fail(KSD_EINVAL, "rosa_credits: negative shape");
  if (lmax < 0 || lmax > 63) return fail(KSD_EINVAL, "rosa_credits: lmax must be in [0, 63]");
  if (T > 65535) return fail(KSD_EINVAL, "rosa_credits: T above 65535 is not supported");
  if (B == 0 || T == 0 || S == 0) return KSD_OK;
  if (!q_bits || !k_bits || !v_bits || !match_j || !grad || !payload || !credits || !payload_partial)
    return fail(KSD_EINVAL, "rosa_credits: null pointer");
  if (!credit_sums) return fail(KSD_EINVAL, "rosa_credits: credit_sums workspace is required");
  const int W = (int)cdiv(T, 32);
  const size_t lds = (4 + 3 * (size_t)W + kCredWaves * (size_t)kCredWave32) * sizeof(uint32_t);
  if (lds > 64 * 1024) return fail(KSD_EINVAL, "rosa_credits: T too large for LDS");
  if (B * S > 0x7fffffff || B * S * cdiv(T, kCredChunk) > 0x7fffffff)
    return fail(KSD_EINVAL, "rosa_credits: too many streams");
  hipStream_t st = (hipStream_t)stream;
  unsigned long long *sums = (unsigned long long *)credit_sums;
  const int n = (int)(B * S);
  hipLaunchKernelGGL(rosa_cred_setup_kernel, dim3((unsigned)n), dim3(256), 3 * (size_t)W * sizeof(uint32_t), st,
                     q_bits, k_bits, v_bits, match_j, grad, payload, S, (int)T, W, lmax, credits,
                     payload_partial, sums);
  if (T >= 2 && lmax >= 1) {  // position 0 has no candidate: T = 1 has no contribution
    if (T <= kBpMaxT) {  // the bit-parallel kernel: one 32-candidate word per lane
      const int nchunks = (int)cdiv(T, kCredChunk);
      const int64_t waves = (int64_t)n * nchunks;
      const int nblk = (int)min(cdiv(waves, kCredWaves), (int64_t)cu_count() * kBpBlocksPerCu);
      hipLaunchKernelGGL(rosa_credits_bp_kernel, dim3((unsigned)nblk), dim3(256), 0, st, q_bits, k_bits,
                         v_bits, match_j, grad, payload, S, (int)T, W, lmax, credits, sums,
                         (unsigned int *)credits + 3, 3 * T, min(n, kCredCounters), n, nchunks,
                         credits_path_override());
    } else {
      hipLaunchKernelGGL(rosa_credits_kernel, dim3((unsigned)n), dim3(256), lds, st, q_bits, k_bits,
                         v_bits, match_j, grad, payload, S, (int)T, W, lmax, credits, sums);
    }
  }
  hipLaunchKernelGGL(rosa_cred_finish_kernel, dim3((unsigned)n), dim3(256), 0, st, credits, sums, (int)T);
  return check_launch("rosa_credits");
}

extern "C" int ksd_rosa_credit_grads(const float *credits, const void *q, const void *k, const void *v,
                                     int dtype, const float *payload_partial, int64_t B, int64_t T,
                                     int64_t S, void *gq, void *gk, void *gv, float *gpayload,
                                     void *stream) {
  if (B < 0 || T < 0 || S < 0) return fail(KSD_EINVAL, "rosa_credit_grads: negative shape");
  if (dtype != KSD_F32 && dtype != KSD_BF16 && dtype != KSD_F16)
    return fail(KSD_ETYPE, "rosa_credit_grads: q/k/v must be float32, bfloat16 or float16");
  if (B == 0 || T == 0 || S == 0) return KSD_OK;
  if (!credits || !q || !k || !v || !payload_partial || !gq || !gk || !gv || !gpayload)
    return fail(KSD_EINVAL, "rosa_credit_grads: null pointer");
  if (B > 65535 || cdiv(T, kCgTile) > 65535) return fail(KSD_EINVAL, "rosa_credit_grads: too large");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)cdiv(S, kCgTile), (unsigned)cdiv(T, kCgTile), (unsigned)B);
  switch (dtype) {
    case KSD_F32: hipLaunchKernelGGL(rosa_credit_grad_kernel<KSD_F32>, grid, dim3(256), 0, st, credits, q, k, v, B, T, S, gq, gk, gv); break;
    case KSD_BF16: hipLaunchKernelGGL(rosa_credit_grad_kernel<KSD_BF16>, grid, dim3(256), 0, st, credits, q, k, v, B, T, S, gq, gk, gv); break;
    default: hipLaunchKernelGGL(rosa_credit_grad_kernel<KSD_F16>, grid, dim3(256), 0, st, credits, q, k, v, B, T, S, gq, gk, gv); break;
  }
  hipLaunchKernelGGL(rosa_payload_grad_kernel, dim3((unsigned)cdiv(S, 256)), dim3(256), 0, st,
                     payload_partial, B, S, gpayload);
  return check_launch("rosa_credit_grads");
}
