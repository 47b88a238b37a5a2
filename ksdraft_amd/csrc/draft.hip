// Kernels of the draft training step around the INT8 surfaces (config 5):
//
//   transfer_cos_kernel / transfer_grad_kernel
//       the transfer-space term of distillation_losses (reference
//       ksdraft/train/__init__.py:79-85): 1 - <normalize(f), e_hat> per row, and its
//       gradient, one wave per row, with no normalized copy of f materialised.
//   inj_up_fwd_kernel / inj_up_bwd_kernel
//       the gated update of the DSpine adjacent injection (reference
//       ksdraft/model/spine.py:62-68): out = z + sigmoid(pre) * u with
//           pre = b + [zd_g | pd_g] . Wc^T   (rank 32 + 32),  u = pd_i . Wiu^T  (rank 32)
//       evaluated from the (M, 96) low-rank operand and the (d, 96) weights in one pass
//       over z (no pre / u / sigmoid tensors), and its backward's elementwise part
//       (dpre = dout u s (1 - s), du = dout s, the same pre and u recomputed).
//   ln_bwd_kernel
//       nn.LayerNorm's backward fused with the residual branch's gradient (the block's
//       x + mixer(ln(x)), reference ksdraft/model/block.py:39-41).
// All arithmetic is fp32 (the float surfaces of the step); the sums run in this file's
// order, so results are within fp32 rounding of torch's, not bit-equal.
#include "ksd_common.h"

namespace ksd {

// ---------------------------------------------------------------- transfer space
// Row r of f (M, d) and e (M, d): dot = f.e and ss = f.f summed by a wave (a lane owns
// d/64 elements, 16-byte loads when d % 4 == 0), combined across lanes by shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <bool VEC>
__global__ __launch_bounds__(256) void transfer_cos_kernel(const float *__restrict__ f,
                                                           const float *__restrict__ e, int M, int d,
                                                           float *__restrict__ cos_out,
                                                           float *__restrict__ nf_out) {
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= M) return;  // wave-uniform
  const float *fr = f + (int64_t)row * d, *er = e + (int64_t)row * d;
  float dot = 0.0f, ss = 0.0f;
  if (VEC) {
    for (int c = lane * 4; c < d; c += 256) {
      const float4 a = *(const float4 *)(fr + c), b = *(const float4 *)(er + c);
      dot += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
  } else {
    for (int c = lane; c < d; c += 64) {
      const float a = fr[c];
      dot += a * er[c];
      ss += a * a;
    }
  }
  dot = wave_sum(dot);
  ss = wave_sum(ss);
  if (lane == 0) {
    const float nf = sqrtf(ss);
    cos_out[row] = dot / fmaxf(nf, 1e-12f);  // F.normalize: x / max(||x||, eps)
    nf_out[row] = nf;
  }
}

// d/df_r of coef * (1 - <f_r / max(|f_r|, eps), e_r>) and, accumulated into ge (or written,
// when `first`), d/de_r = -coef * f_r / max(|f_r|, eps). For |f_r| > eps the first is
// -coef (e_r - cos_r f_r / |f_r|) / |f_r|; at or below eps the norm is the constant eps.
// coef is a device scalar (the upstream gradient times the loss weight over M rows).
template <bool VEC>
__global__ __launch_bounds__(256) void transfer_grad_kernel(
    const float *__restrict__ f, const float *__restrict__ e, const float *__restrict__ cosv,
    const float *__restrict__ nfv, const float *__restrict__ coef, int M, int d,
    float *__restrict__ df, float *__restrict__ ge, int first) {
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= M) return;
  const float nf = nfv[row], cs = cosv[row], k = *coef;
  const bool big = nf > 1e-12f;
  const float inv = 1.0f / fmaxf(nf, 1e-12f);
  const float a = -k * inv, b = big ? k * cs * inv * inv : 0.0f;  // df = a e + b f
  const int64_t o = (int64_t)row * d;
  if (VEC) {
    for (int c = lane * 4; c < d; c += 256) {
      const float4 fv = *(const float4 *)(f + o + c), ev = *(const float4 *)(e + o + c);
      *(float4 *)(df + o + c) = make_float4(a * ev.x + b * fv.x, a * ev.y + b * fv.y,
                                            a * ev.z + b * fv.z, a * ev.w + b * fv.w);
      float4 g = first ? make_float4(0.f, 0.f, 0.f, 0.f) : *(const float4 *)(ge + o + c);
      g.x += a * fv.x;
      g.y += a * fv.y;
      g.z += a * fv.z;
      g.w += a * fv.w;
      *(float4 *)(ge + o + c) = g;
    }
  } else {
    for (int c = lane; c < d; c += 64) {
      const float fv = f[o + c], ev = e[o + c];
      df[o + c] = a * ev + b * fv;
      ge[o + c] = (first ? 0.0f : ge[o + c]) + a * fv;
    }
  }
}

// ---------------------------------------------------------------- injection update
// Block = 256 threads = 256 consecutive columns c of d, walking RB rows. A thread keeps its
// column's 96 weights [Wc[c, 0:64] | Wiu[c, 0:32]] and b[c] in registers; the block's RB
// rows of the (M, 96) operand [zd_g | pd_g | pd_i] sit in LDS and are read as broadcasts.
constexpr int kInjRank = 96, kInjRows = 64;

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

template <bool BWD>
__global__ __launch_bounds__(256) void inj_up_kernel(
    const float *__restrict__ zs, const float *__restrict__ wc, const float *__restrict__ wiu,
    const float *__restrict__ bias, const float *__restrict__ zin, const float *__restrict__ gout,
    int M, int d, float *__restrict__ out, float *__restrict__ dpre, float *__restrict__ du) {
  __shared__ __attribute__((aligned(16))) float srow[kInjRows * kInjRank];
  const int c = (int)blockIdx.x * 256 + (int)threadIdx.x;
  const int r0 = (int)blockIdx.y * kInjRows;
  const int nr = min(kInjRows, M - r0);
  for (int i = threadIdx.x; i < nr * kInjRank / 4; i += 256)
    ((float4 *)srow)[i] = ((const float4 *)(zs + (int64_t)r0 * kInjRank))[i];
  __syncthreads();
  if (c >= d) return;  // after the block's only barrier
  float w[kInjRank];
#pragma unroll
  for (int k = 0; k < 64; k += 4) {
    const float4 v = *(const float4 *)(wc + (int64_t)c * 64 + k);
    w[k] = v.x; w[k + 1] = v.y; w[k + 2] = v.z; w[k + 3] = v.w;
  }
#pragma unroll
  for (int k = 0; k < 32; k += 4) {
    const float4 v = *(const float4 *)(wiu + (int64_t)c * 32 + k);
    w[64 + k] = v.x; w[65 + k] = v.y; w[66 + k] = v.z; w[67 + k] = v.w;
  }
  const float bc = bias ? bias[c] : 0.0f;
  for (int i = 0; i < nr; ++i) {
    const float4 *sr = (const float4 *)(srow + i * kInjRank);
    // four independent partial sums per float4 lane slot: short dependency chains
    float pa[4] = {0.f, 0.f, 0.f, 0.f}, ua[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k4 = 0; k4 < 16; ++k4) {
      const float4 v = sr[k4];
      pa[0] = fmaf(v.x, w[4 * k4], pa[0]);
      pa[1] = fmaf(v.y, w[4 * k4 + 1], pa[1]);
      pa[2] = fmaf(v.z, w[4 * k4 + 2], pa[2]);
      pa[3] = fmaf(v.w, w[4 * k4 + 3], pa[3]);
    }
#pragma unroll
    for (int k4 = 16; k4 < 24; ++k4) {
      const float4 v = sr[k4];
      ua[0] = fmaf(v.x, w[4 * k4], ua[0]);
      ua[1] = fmaf(v.y, w[4 * k4 + 1], ua[1]);
      ua[2] = fmaf(v.z, w[4 * k4 + 2], ua[2]);
      ua[3] = fmaf(v.w, w[4 * k4 + 3], ua[3]);
    }
    const float pre = bc + ((pa[0] + pa[1]) + (pa[2] + pa[3]));
    const float u = (ua[0] + ua[1]) + (ua[2] + ua[3]);
    const float s = sigmoid_f(pre);
    const int64_t o = (int64_t)(r0 + i) * d + c;
    if constexpr (!BWD) {
      out[o] = zin[o] + s * u;
    } else {
      const float g = gout[o];
      dpre[o] = g * u * (s * (1.0f - s));
      du[o] = g * s;
    }
  }
}

// ---------------------------------------------------------------- layer norm backward
// nn.LayerNorm's backward (reference ksdraft/model/block.py:27-41) for rows of x (M, d)
// with the per-row mean and rstd of the forward, fused with the gradient of the residual
// branch that reads the same x (the block's x + mixer(ln(x))):
//   xhat = (x - mean) rstd,  g = dy w,
//   dx   = rstd (g - xhat mean(g xhat) - mean(g)) + dres,
// and the block's share of dw = sum dy xhat, db = sum dy over its rows, written as
// partials (n_blocks, 2, d) that the caller adds (the four waves' sums added in wave
// order). A wave walks kLnBwdRows / 4 rows; a lane owns NQ groups of 4 columns (d = 256 NQ,
// 16-byte access), keeping its columns' dw / db sums in registers.
constexpr int kLnBwdRows = 16;  // rows per block

template <int NQ, bool RES>
__global__ __launch_bounds__(256) void ln_bwd_kernel(
    const float *__restrict__ x, const float *__restrict__ dy, const float *__restrict__ dres,
    const float *__restrict__ mean, const float *__restrict__ rstd, const float *__restrict__ w,
    int M, float *__restrict__ dx, float *__restrict__ part) {
  constexpr int d = 256 * NQ, NV = 4 * NQ;
  __shared__ __attribute__((aligned(16))) float red[2][d];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float aw[NV], ab[NV], wv[NV];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const float4 v = *(const float4 *)(w + q * 256 + lane * 4);
    wv[4 * q] = v.x; wv[4 * q + 1] = v.y; wv[4 * q + 2] = v.z; wv[4 * q + 3] = v.w;
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    aw[i] = 0.0f;
    ab[i] = 0.0f;
  }
  constexpr float inv_d = 1.0f / (float)d;
  const int r_end = min((int)(blockIdx.x + 1) * kLnBwdRows, M);
  for (int r = (int)blockIdx.x * kLnBwdRows + wave; r < r_end; r += 4) {  // wave-uniform
    const int64_t o = (int64_t)r * d + lane * 4;
    const float mu = mean[r], rs = rstd[r];
    float xh[NV], gg[NV];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const float4 a = *(const float4 *)(x + o + q * 256), b = *(const float4 *)(dy + o + q * 256);
      const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = 4 * q + k;
        xh[i] = (av[k] - mu) * rs;
        gg[i] = bv[k] * wv[i];
        s1 += gg[i] * xh[i];
        s2 += gg[i];
        aw[i] += bv[k] * xh[i];
        ab[i] += bv[k];
      }
    }
    s1 = wave_sum(s1) * inv_d;
    s2 = wave_sum(s2) * inv_d;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      float4 rv = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (RES) rv = *(const float4 *)(dres + o + q * 256);
      const float rr[4] = {rv.x, rv.y, rv.z, rv.w};
      float out[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = 4 * q + k;
        out[k] = rs * (gg[i] - xh[i] * s1 - s2) + rr[k];
      }
      *(float4 *)(dx + o + q * 256) = make_float4(out[0], out[1], out[2], out[3]);
    }
  }
  // the block's column sums, the four waves added in order
#pragma unroll 1
  for (int wv_ = 0; wv_ < 4; ++wv_) {
    if (wave == wv_) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        float4 *p0 = (float4 *)(red[0] + q * 256 + lane * 4), *p1 = (float4 *)(red[1] + q * 256 + lane * 4);
        float4 a = make_float4(aw[4 * q], aw[4 * q + 1], aw[4 * q + 2], aw[4 * q + 3]);
        float4 b = make_float4(ab[4 * q], ab[4 * q + 1], ab[4 * q + 2], ab[4 * q + 3]);
        if (wv_ > 0) {
          const float4 a0 = *p0, b0 = *p1;
          a = make_float4(a0.x + a.x, a0.y + a.y, a0.z + a.z, a0.w + a.w);
          b = make_float4(b0.x + b.x, b0.y + b.y, b0.z + b.z, b0.w + b.w);
        }
        *p0 = a;
        *p1 = b;
      }
    }
    __syncthreads();
  }
  for (int idx = threadIdx.x; idx < 2 * d; idx += 256)
    part[(int64_t)blockIdx.x * 2 * d + idx] = red[idx / d][idx % d];
}

}  // namespace ksd

using namespace ksd;

extern "C" int ksd_transfer_cos(const float *f, const float *e_hat, int64_t M, int64_t d,
                                float *cos_out, float *norm_out, void *stream) {
  if (M < 0 || d < 0) return fail(KSD_EINVAL, "transfer_cos: negative shape");
  if (M == 0 || d == 0) return KSD_OK;
  if (!f || !e_hat || !cos_out || !norm_out) return fail(KSD_EINVAL, "transfer_cos: null pointer");
  if (M > 0x7ffffff0LL || d > 0x7fffffffLL) return fail(KSD_EINVAL, "transfer_cos: too large");
  const bool vec = d % 4 == 0 && ((uintptr_t)f % 16) == 0 && ((uintptr_t)e_hat % 16) == 0;
  const dim3 grid((unsigned)cdiv(M, 4));
  hipStream_t st = (hipStream_t)stream;
  if (vec)
    hipLaunchKernelGGL(transfer_cos_kernel<true>, grid, dim3(256), 0, st, f, e_hat, (int)M, (int)d, cos_out, norm_out);
  else
    hipLaunchKernelGGL(transfer_cos_kernel<false>, grid, dim3(256), 0, st, f, e_hat, (int)M, (int)d, cos_out, norm_out);
  return check_launch("transfer_cos");
}

extern "C" int ksd_transfer_grad(const float *f, const float *e_hat, const float *cos_in,
                                 const float *norm_in, const float *coef, int64_t M, int64_t d,
                                 float *df, float *grad_e, int first, void *stream) {
  if (M < 0 || d < 0) return fail(KSD_EINVAL, "transfer_grad: negative shape");
  if (M == 0 || d == 0) return KSD_OK;
  if (!f || !e_hat || !cos_in || !norm_in || !coef || !df || !grad_e)
    return fail(KSD_EINVAL, "transfer_grad: null pointer");
  if (M > 0x7ffffff0LL || d > 0x7fffffffLL) return fail(KSD_EINVAL, "transfer_grad: too large");
  const bool vec = d % 4 == 0 && ((uintptr_t)f % 16) == 0 && ((uintptr_t)e_hat % 16) == 0 &&
                   ((uintptr_t)df % 16) == 0 && ((uintptr_t)grad_e % 16) == 0;
  const dim3 grid((unsigned)cdiv(M, 4));
  hipStream_t st = (hipStream_t)stream;
  if (vec)
    hipLaunchKernelGGL(transfer_grad_kernel<true>, grid, dim3(256), 0, st, f, e_hat, cos_in, norm_in,
                       coef, (int)M, (int)d, df, grad_e, first);
  else
    hipLaunchKernelGGL(transfer_grad_kernel<false>, grid, dim3(256), 0, st, f, e_hat, cos_in, norm_in,
                       coef, (int)M, (int)d, df, grad_e, first);
  return check_launch("transfer_grad");
}

static int inj_checks(const char *who, const float *zs, const float *wc, const float *wiu,
                      int64_t M, int64_t d) {
  if (M < 0 || d < 0) return fail(KSD_EINVAL, "%s: negative shape", who);
  if (!zs || !wc || !wiu) return fail(KSD_EINVAL, "%s: null pointer", who);
  if (((uintptr_t)zs | (uintptr_t)wc | (uintptr_t)wiu) % 16)
    return fail(KSD_EINVAL, "%s: the rank operand and weights must be 16-byte aligned", who);
  if (M > 0x7fffffffLL - kInjRows || d > (1LL << 24)) return fail(KSD_EINVAL, "%s: too large", who);
  return KSD_OK;
}

extern "C" int ksd_injection_update(const float *zs, const float *wc, const float *wiu,
                                    const float *bias, const float *z, int64_t M, int64_t d,
                                    float *out, void *stream) {
  int rc = inj_checks("injection_update", zs, wc, wiu, M, d);
  if (rc) return rc;
  if (M == 0 || d == 0) return KSD_OK;
  if (!z || !out) return fail(KSD_EINVAL, "injection_update: null pointer");
  const dim3 grid((unsigned)cdiv(d, 256), (unsigned)cdiv(M, kInjRows));
  hipLaunchKernelGGL(inj_up_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, zs, wc, wiu, bias,
                     z, (const float *)nullptr, (int)M, (int)d, out, (float *)nullptr, (float *)nullptr);
  return check_launch("injection_update");
}

extern "C" int ksd_injection_update_backward(const float *zs, const float *wc, const float *wiu,
                                             const float *bias, const float *grad_out, int64_t M,
                                             int64_t d, float *dpre, float *du, void *stream) {
  int rc = inj_checks("injection_update_backward", zs, wc, wiu, M, d);
  if (rc) return rc;
  if (M == 0 || d == 0) return KSD_OK;
  if (!grad_out || !dpre || !du) return fail(KSD_EINVAL, "injection_update_backward: null pointer");
  const dim3 grid((unsigned)cdiv(d, 256), (unsigned)cdiv(M, kInjRows));
  hipLaunchKernelGGL(inj_up_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, zs, wc, wiu, bias,
                     (const float *)nullptr, grad_out, (int)M, (int)d, (float *)nullptr, dpre, du);
  return check_launch("injection_update_backward");
}


extern "C" int ksd_layernorm_backward_blocks(int64_t M, int64_t *n_blocks) {
  if (!n_blocks || M < 0) return fail(KSD_EINVAL, "layernorm_backward_blocks: bad argument");
  *n_blocks = cdiv(M, kLnBwdRows);
  return KSD_OK;
}

extern "C" int ksd_layernorm_backward(const float *x, const float *dy, const float *dres,
                                      const float *mean, const float *rstd, const float *weight,
                                      int64_t M, int64_t d, float *dx, float *partials,
                                      void *stream) {
  if (M < 0 || d < 0) return fail(KSD_EINVAL, "layernorm_backward: negative shape");
  if (M == 0 || d == 0) return KSD_OK;
  if (d % 256 || d > 2048)
    return fail(KSD_EINVAL, "layernorm_backward: d must be a multiple of 256, at most 2048");
  if (!x || !dy || !mean || !rstd || !weight || !dx || !partials)
    return fail(KSD_EINVAL, "layernorm_backward: null pointer");
  if (((uintptr_t)x | (uintptr_t)dy | (uintptr_t)dres | (uintptr_t)weight | (uintptr_t)dx) % 16)
    return fail(KSD_EINVAL, "layernorm_backward: rows must be 16-byte aligned");
  if (M > 0x7fffffffLL - kLnBwdRows) return fail(KSD_EINVAL, "layernorm_backward: too large");
  const dim3 grid((unsigned)cdiv(M, kLnBwdRows));
  hipStream_t st = (hipStream_t)stream;
#define KSD_LNB(NQ)                                                                                 \
  if (dres)                                                                                        \
    hipLaunchKernelGGL((ln_bwd_kernel<NQ, true>), grid, dim3(256), 0, st, x, dy, dres, mean, rstd, \
                       weight, (int)M, dx, partials);                                              \
  else                                                                                             \
    hipLaunchKernelGGL((ln_bwd_kernel<NQ, false>), grid, dim3(256), 0, st, x, dy, dres, mean, rstd,\
                       weight, (int)M, dx, partials);
  switch (d / 256) {
    case 1: KSD_LNB(1) break;
    case 2: KSD_LNB(2) break;
    case 3: KSD_LNB(3) break;
    case 4: KSD_LNB(4) break;
    case 5: KSD_LNB(5) break;
    case 6: KSD_LNB(6) break;
    case 7: KSD_LNB(7) break;
    default: KSD_LNB(8) break;
  }
#undef KSD_LNB
  return check_launch("layernorm_backward");
}
