// W8A8 GS-group GEMM for gfx950 on the int8 matrix cores.
//
//   Y[m,n] = sum_g float(P_g[m,n]) * (sa[m,g] * sw[n,g]),  P_g = sum_{k in g} A[m,k] W[n,k]
//
// computed in the ordered contract acc = fmaf(float(P_g), sa*sw, acc), g = 0,1,...
// (the per-group rescale of reference ksdraft/kernels/gemm.py:42-45; sa*sw is exact in
// fp32 because both factors are fp16 values, and float(P_g) is exact because
// |P_g| <= 128*127^2 < 2^24).
//
// Layout "NT": A (M,K) and W (N,K) both K-contiguous int8; scales (rows, K/group) fp16.
// Block tile 128x128, K step 128 (a whole number of groups), 4 waves each owning a
// 64x64 sub-tile = 2x2 MFMA 32x32 tiles. A/W tiles are staged global -> registers ->
// LDS (double buffered, one barrier per K step); the LDS rows are 128 bytes and the
// 16-byte chunk index is XOR-swizzled with (row & 7) so that the ds_read_b128 operand
// fetches of 8 consecutive rows hit 8 distinct bank groups.
#include "ksd_common.h"

namespace ksd {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 128;

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * BK + ((chunk ^ (row & 7)) << 4);
}

// MODE 0: fp32 epilogue into Y with output type OUT (and optional bias).
// MODE 1: export the int32 group partials P_g to `partials` (G, M, N).
template <int GROUP, int OUT, bool BIAS, int MODE>
__global__ __launch_bounds__(256, 2) void gemm_nt_kernel(
    const int8_t *__restrict__ A, const uint16_t *__restrict__ AS,
    const int8_t *__restrict__ W, const uint16_t *__restrict__ WS, int M, int N, int K,
    int tiles_n, const float *__restrict__ bias, void *__restrict__ Y,
    int32_t *__restrict__ partials) {
  constexpr int GPT = BK / GROUP;  // groups per K step
  constexpr int MPG = GROUP / 32;  // 32-deep MFMAs per group
  __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * BK];
  __shared__ __attribute__((aligned(16))) int8_t sW[2][BN * BK];
  __shared__ __attribute__((aligned(16))) float sSA[2][GPT][BM];
  __shared__ __attribute__((aligned(16))) float sSW[2][GPT][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // Workgroups are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8), each
  // with its own L2. Renumber so that XCD x owns a contiguous range of tiles in
  // row-major tile order: the tiles sharing an A row panel then share one L2.
  int bid = blockIdx.x;
  {
    const int nb = gridDim.x, per = nb / 8, rem = nb % 8, x = bid % 8, i = bid / 8;
    // XCD x receives per (+1 if x < rem) blocks; they take tiles [start_x, start_x + cnt)
    bid = x * per + min(x, rem) + i;
  }
  const int tm = bid / tiles_n, tn = bid % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int G = K / GROUP;
  const int KT = K / BK;

  // global -> register staging: 1024 16-byte chunks per operand tile, 4 per thread
  const int lrow = tid >> 3, lch = tid & 7;
  const int8_t *gA[4];
  const int8_t *gW[4];
  int soff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = lrow + 32 * i;
    gA[i] = A + (int64_t)min(m0 + r, M - 1) * K + lch * 16;
    gW[i] = W + (int64_t)min(n0 + r, N - 1) * K + lch * 16;
    soff[i] = swz(r, lch);
  }
  // scale staging: threads 0..127 own A rows, 128..255 own W rows
  const bool sc_a = tid < 128;
  const int sc_r = tid & 127;
  const uint16_t *gS = sc_a ? AS + (int64_t)min(m0 + sc_r, M - 1) * G
                            : WS + (int64_t)min(n0 + sc_r, N - 1) * G;

  v4i ra[4], rw[4];
  uint16_t rs[GPT];  // raw fp16 bits: converting here would force an early vmcnt wait
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = *(const v4i *)(gA[i] + kt * BK);
      rw[i] = *(const v4i *)(gW[i] + kt * BK);
    }
    if (MODE == 0) {
#pragma unroll
      for (int g = 0; g < GPT; ++g) rs[g] = gS[kt * GPT + g];
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(v4i *)(&sA[buf][soff[i]]) = ra[i];
      *(v4i *)(&sW[buf][soff[i]]) = rw[i];
    }
    if (MODE == 0) {
#pragma unroll
      for (int g = 0; g < GPT; ++g) {
        if (sc_a) sSA[buf][g][sc_r] = f16_to_f32(rs[g]);
        else sSW[buf][g][sc_r] = f16_to_f32(rs[g]);
      }
    }
  };

  float acc[2][2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  gload(0);
  lstore(0);
  __syncthreads();

  const int half = lane >> 5, l32 = lane & 31;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) {
      v16i p[2][2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) p[i][j] = (v16i){};
#pragma unroll
      for (int kk = 0; kk < MPG; ++kk) {
        const int kc = (gi * MPG + kk) * 2 + half;
        v4i a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int row = wm * 64 + i * 32 + l32;
          a[i] = *(const v4i *)(&sA[cur][swz(row, kc)]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = wn * 64 + j * 32 + l32;
          b[j] = *(const v4i *)(&sW[cur][swz(col, kc)]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            p[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], p[i][j], 0, 0, 0);
      }
      if (MODE == 0) {
        float sw[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) sw[j] = sSW[cur][gi][wn * 64 + j * 32 + l32];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 sa4 =
                *(const float4 *)(&sSA[cur][gi][wm * 64 + i * 32 + q * 8 + half * 4]);
            const float sa[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4)
#pragma unroll
              for (int j = 0; j < 2; ++j) {
                const int e = q * 4 + e4;
                acc[i][j][e] = fmaf((float)p[i][j][e], sa[e4] * sw[j], acc[i][j][e]);
              }
          }
      } else {
        const int g = kt * GPT + gi;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
              const int col = n0 + wn * 64 + j * 32 + l32;
              if (row < M && col < N)
                partials[((int64_t)g * M + row) * N + col] = p[i][j][e];
            }
      }
    }
    if (kt + 1 < KT) lstore(cur ^ 1);
    __syncthreads();
  }

  if (MODE == 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + l32;
      if (col >= N) continue;
      const float b = BIAS ? bias[col] : 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
          if (row >= M) continue;
          float v = acc[i][j][e];
          if (BIAS) v = v + b;
          store_out<OUT>(Y, (int64_t)row * N + col, v);
        }
    }
  }
}

template <int GROUP, int OUT, bool BIAS>
static void launch_gemm(const int8_t *a, const uint16_t *as, const int8_t *w,
                        const uint16_t *ws, int M, int N, int K, const float *bias, void *y,
                        hipStream_t st) {
  const int tn = (N + BN - 1) / BN, tm = (M + BM - 1) / BM;
  gemm_nt_kernel<GROUP, OUT, BIAS, 0><<<dim3(tm * tn), dim3(256), 0, st>>>(
      a, as, w, ws, M, N, K, tn, bias, y, nullptr);
}

template <int GROUP, int OUT>
static void launch_gemm_b(const int8_t *a, const uint16_t *as, const int8_t *w,
                          const uint16_t *ws, int M, int N, int K, const float *bias, void *y,
                          hipStream_t st) {
  if (bias) launch_gemm<GROUP, OUT, true>(a, as, w, ws, M, N, K, bias, y, st);
  else launch_gemm<GROUP, OUT, false>(a, as, w, ws, M, N, K, bias, y, st);
}

template <int GROUP>
static int launch_gemm_o(const int8_t *a, const uint16_t *as, const int8_t *w,
                         const uint16_t *ws, int M, int N, int K, const float *bias, void *y,
                         int y_dtype, hipStream_t st) {
  switch (y_dtype) {
    case KSD_F32: launch_gemm_b<GROUP, KSD_F32>(a, as, w, ws, M, N, K, bias, y, st); break;
    case KSD_BF16: launch_gemm_b<GROUP, KSD_BF16>(a, as, w, ws, M, N, K, bias, y, st); break;
    case KSD_F16: launch_gemm_b<GROUP, KSD_F16>(a, as, w, ws, M, N, K, bias, y, st); break;
    case KSD_F16_SAT: launch_gemm_b<GROUP, KSD_F16_SAT>(a, as, w, ws, M, N, K, bias, y, st); break;
    default: return fail(KSD_ETYPE, "w8a8_gemm: unsupported output dtype %d", y_dtype);
  }
  return check_launch("w8a8_gemm_nt");
}

static int gemm_checks(const int8_t *a, const int8_t *w, int64_t M, int64_t N, int64_t K,
                       int group) {
  if (!valid_group(group)) return fail(KSD_EINVAL, "group must be 32, 64 or 128, got %d", group);
  if (M < 0 || N < 0 || K < 0) return fail(KSD_EINVAL, "negative GEMM shape");
  if (K % BK != 0) return fail(KSD_EINVAL, "w8a8_gemm: K=%lld must be a multiple of 128", (long long)K);
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL ||
      ((M + BM - 1) / BM) * ((N + BN - 1) / BN) > 0x7fffffffLL)
    return fail(KSD_EINVAL, "w8a8_gemm: shape too large");
  if (((uintptr_t)a) % 16 != 0 || ((uintptr_t)w) % 16 != 0)
    return fail(KSD_EINVAL, "w8a8_gemm: operands must be 16-byte aligned");
  return KSD_OK;
}

}  // namespace ksd

using namespace ksd;

extern "C" int ksd_w8a8_gemm_nt(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                                const uint16_t *w_scales, int64_t M, int64_t N, int64_t K,
                                int group, const float *bias, void *y, int y_dtype,
                                void *stream) {
  int rc = gemm_checks(a, w, M, N, K, group);
  if (rc != KSD_OK) return rc;
  if (M == 0 || N == 0 || K == 0) return KSD_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (group) {
    case 32: return launch_gemm_o<32>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
    case 64: return launch_gemm_o<64>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
    default: return launch_gemm_o<128>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
  }
}

extern "C" int ksd_w8a8_group_partials(const int8_t *a, const int8_t *w, int64_t M, int64_t N,
                                       int64_t K, int group, int32_t *partials,
                                       void *stream) {
  int rc = gemm_checks(a, w, M, N, K, group);
  if (rc != KSD_OK) return rc;
  if (M == 0 || N == 0 || K == 0) return KSD_OK;
  hipStream_t st = (hipStream_t)stream;
  const int tn = (int)((N + BN - 1) / BN), tm = (int)((M + BM - 1) / BM);
  const dim3 grid(tm * tn), block(256);
  switch (group) {
    case 32: gemm_nt_kernel<32, KSD_F32, false, 1><<<grid, block, 0, st>>>(a, nullptr, w, nullptr, (int)M, (int)N, (int)K, tn, nullptr, nullptr, partials); break;
    case 64: gemm_nt_kernel<64, KSD_F32, false, 1><<<grid, block, 0, st>>>(a, nullptr, w, nullptr, (int)M, (int)N, (int)K, tn, nullptr, nullptr, partials); break;
    default: gemm_nt_kernel<128, KSD_F32, false, 1><<<grid, block, 0, st>>>(a, nullptr, w, nullptr, (int)M, (int)N, (int)K, tn, nullptr, nullptr, partials); break;
  }
  return check_launch("w8a8_group_partials");
}
