// W8A8 GS-group GEMM for gfx950 on the int8 matrix cores.
//
//   Y[m,n] = sum_g float(P_g[m,n]) * (sa[m,g] * sw[n,g]),  P_g = sum_{k in g} A[m,k] W[n,k]
//
// computed in the ordered contract acc = fmaf(float(P_g), sa*sw, acc), g = 0,1,...
// (the per-group rescale of reference ksdraft/kernels/gemm.py:42-45). sa*sw is exact in
// fp32 (both factors are fp16 values) and float(P_g) is exact (|P_g| <= 128*127^2 < 2^24).
//
// Layout "NT": A (M,K) and W (N,K) both K-contiguous int8; scales (rows, K/group) fp16.
//
// Two kernels share the tile geometry: gemm_g128_kernel (below, group 128: the
// production path) and gemm_nt_kernel (groups 32 and 64, and the int32 partials export).
//
// gemm_nt_kernel structure (one 512-thread workgroup per CU, persistent):
//   * 128x128 output tiles; every workgroup owns a contiguous chunk of tiles in row-major
//     order, and the workgroups of one XCD (dispatched round-robin over 8 XCDs) own
//     neighbouring chunks, so tiles sharing an A row panel share one L2.
//   * K advances 128 per step through a 3-slot LDS ring filled by global_load_lds_dwordx4
//     (no VGPR staging); the DMA for step q+2 is issued at step q into the slot every
//     wave finished reading at step q-1. Each wave waits only for its own DMA of the
//     current step (s_waitcnt vmcnt = one later stage), then a bare s_barrier.
//   * 8 waves as 2 (M) x 4 (N), each owning 64x32 = two 32x32 MFMA tiles.
//   * Per group: 4 x v_mfma_i32_32x32x32_i8 per tile give the exact int32 partial; the
//     scale products sa[m]*sw[n] of the whole 32x32 tile come from one
//     v_mfma_f32_32x32x8_f16 outer product (a single non-zero k slot, so exact); the VALU
//     then does cvt + fma per element. The int32 partials are double buffered so the
//     MFMAs of group g overlap the VALU epilogue of group g-1.
//   * LDS rows are 128 bytes; the 16-byte chunk index is XOR-swizzled with (row & 7).
#include "ksd_common.h"

namespace ksd {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

#define KSD_LDS(p) ((__attribute__((address_space(3))) void *)(p))
// s_waitcnt vmcnt(n) lgkmcnt(0) as inline asm with a memory clobber: a hard compiler
// barrier, so no DMA of an earlier step can be sunk below the wait (the builtin is not a
// memory barrier for the optimizer). lgkmcnt(0): this wave's LDS reads of the slot about
// to be refilled have returned before it enters the barrier.
#define KSD_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(" #n ") lgkmcnt(0)" ::: "memory")

constexpr int BM = 128, BN = 128, BK = 128, NSLOT = 4, NTHREADS = 512;

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * BK + ((chunk ^ (row & 7)) << 4);
}

// LDS-DMA loads as inline asm (M0 = LDS destination, set in the same statement). The
// compiler does not model these as pending LDS writes, so it does not add its own
// vmcnt(0) before LDS reads; the kernel's explicit KSD_WAIT_VM waits carry correctness.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)KSD_LDS(p);
}
// `lds` must be wave-uniform (kept in an SGPR).
__device__ __forceinline__ void dma16(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma2(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_ushort %0, off"
               :: "v"(g), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// MODE 0: fp32 epilogue into Y (output type OUT, optional bias).
// MODE 1: export the int32 group partials P_g to `partials` (G, M, N) (test path).
template <int GROUP, int OUT, bool BIAS, int MODE>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_nt_kernel(
    const int8_t *__restrict__ A, const uint16_t *__restrict__ AS,
    const int8_t *__restrict__ W, const uint16_t *__restrict__ WS, int M, int N, int K,
    int tiles_n, int ntiles, const float *__restrict__ bias, void *__restrict__ Y,
    int32_t *__restrict__ partials) {
  constexpr int GPT = BK / GROUP;   // groups per K step
  constexpr int MPG = GROUP / 32;   // 32-deep int8 MFMAs per group
  __shared__ __attribute__((aligned(16))) int8_t sA[NSLOT][BM * BK];
  __shared__ __attribute__((aligned(16))) int8_t sW[NSLOT][BN * BK];
  // fp16 scales in the low half of dword slots (the ushort DMA writes one dword per
  // lane): [0,128) rows of A, [128,256) rows of W
  __shared__ __attribute__((aligned(16))) uint32_t sS[NSLOT][GPT][256];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3, half = lane >> 5, l32 = lane & 31;
  const int G = K / GROUP, KT = K / BK;

  int lb;  // logical block: consecutive on one XCD
  {
    const int nb = gridDim.x, per = nb / 8, rem = nb % 8, x = blockIdx.x % 8, i = blockIdx.x / 8;
    lb = x * per + min(x, rem) + i;
  }
  const int t_begin = (int)((int64_t)ntiles * lb / gridDim.x);
  const int t_end = (int)((int64_t)ntiles * (lb + 1) / gridDim.x);
  const int total = (t_end - t_begin) * KT;
  if (total == 0) return;

  // DMA issue state for the stage being prefetched: per-lane source pointers of this
  // wave's two A rows, two W rows and one scale row, advanced by one K step per issue
  // and re-based only when the issue cursor crosses into the next tile.
  const int ii0 = wave * 2, w4 = wave & 3;
  const int drow0 = ii0 * 8 + (lane >> 3), drow1 = drow0 + 8;
  const int dchunk0 = ((lane & 7) ^ (drow0 & 7)) << 4, dchunk1 = ((lane & 7) ^ (drow1 & 7)) << 4;
  const int srow = (w4 & 1) * 64 + lane;
  const bool s_isA = w4 < 2;
  // wave-uniform LDS destinations, moved to SGPRs once
  const uint32_t ldsA = __builtin_amdgcn_readfirstlane(lds_addr(&sA[0][0]) + ii0 * 1024);
  const uint32_t ldsW = __builtin_amdgcn_readfirstlane(lds_addr(&sW[0][0]) + ii0 * 1024);
  const uint32_t ldsS = __builtin_amdgcn_readfirstlane(
      lds_addr(&sS[0][0][0]) + ((s_isA ? 0 : 128) + (w4 & 1) * 64) * 4);
  const int8_t *pa0, *pa1, *pw0, *pw1;
  const uint16_t *ps;
  int is_tile = t_begin, is_kt = 0, is_slot = 0;
  auto rebase = [&]() {
    const int m0 = (is_tile / tiles_n) * BM, n0 = (is_tile % tiles_n) * BN;
    pa0 = A + (int64_t)min(m0 + drow0, M - 1) * K + dchunk0;
    pa1 = A + (int64_t)min(m0 + drow1, M - 1) * K + dchunk1;
    pw0 = W + (int64_t)min(n0 + drow0, N - 1) * K + dchunk0;
    pw1 = W + (int64_t)min(n0 + drow1, N - 1) * K + dchunk1;
    ps = s_isA ? AS + (int64_t)min(m0 + srow, M - 1) * G : WS + (int64_t)min(n0 + srow, N - 1) * G;
  };
  rebase();
  auto issue = [&]() {
    const uint32_t so = (uint32_t)is_slot * (BM * BK);
    dma16(pa0, ldsA + so);
    dma16(pa1, ldsA + so + 1024);
    dma16(pw0, ldsW + so);
    dma16(pw1, ldsW + so + 1024);
    if (MODE == 0) {
#pragma unroll
      for (int g = 0; g < GPT; ++g) dma2(ps + g, ldsS + (uint32_t)(is_slot * GPT + g) * 1024);
    }
    pa0 += BK; pa1 += BK; pw0 += BK; pw1 += BK; ps += GPT;
    is_slot = is_slot == NSLOT - 1 ? 0 : is_slot + 1;
    if (++is_kt == KT) {
      is_kt = 0;
      if (++is_tile < t_end) rebase();
    }
  };

  // Operand fragments of group gi: 2 A tiles x MPG and 1 W tile x MPG (ds_read_b128 each)
  struct Frags { v4i a[MPG][2]; v4i b[MPG]; uint32_t sa[2], sw; };
  auto load_frags = [&](int slot, int gi, Frags &f) {
#pragma unroll
    for (int kk = 0; kk < MPG; ++kk) {
      const int kc = (gi * MPG + kk) * 2 + half;
      f.b[kk] = *(const v4i *)(&sW[slot][swz(wn * 32 + l32, kc)]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        f.a[kk][i] = *(const v4i *)(&sA[slot][swz(wm * 64 + i * 32 + l32, kc)]);
    }
    if (MODE == 0) {
      const uint32_t *ss = sS[slot][gi];
      f.sw = ss[128 + wn * 32 + l32];
      f.sa[0] = ss[wm * 64 + l32];
      f.sa[1] = ss[wm * 64 + 32 + l32];
    }
  };
  // int32 partials of the two 32x32 tiles
  auto mfma_group = [&](const Frags &f, v16i (&p)[2]) {
    p[0] = (v16i){};
    p[1] = (v16i){};
#pragma unroll
    for (int kk = 0; kk < MPG; ++kk)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        p[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[kk][i], f.b[kk], p[i], 0, 0, 0);
  };
  // s[i] = sa (x) sw for the two tiles: an fp16 MFMA whose only non-zero k slot is 0
  // (lanes 32-63 carry k = 4..7 and supply zeros), so every product is exact in fp32
  auto scale_group = [&](const Frags &f, v16f (&s)[2]) {
    const _Float16 zero = (_Float16)0.0f;
    const _Float16 swv = half ? zero : __builtin_bit_cast(_Float16, (uint16_t)f.sw);
    const v4h bs = {swv, zero, zero, zero};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const _Float16 sav = half ? zero : __builtin_bit_cast(_Float16, (uint16_t)f.sa[i]);
      const v4h as = {sav, zero, zero, zero};
      s[i] = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs, (v16f){}, 0, 0, 0);
    }
  };

  v16f acc[2];
  acc[0] = (v16f){};
  acc[1] = (v16f){};
  auto epilogue = [&](const v16i (&p)[2], const v16f (&s)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] = fmaf((float)p[i][e], s[i][e], acc[i][e]);
  };
  // Stores the finished tile: full tiles without per-element bounds checks, edge tiles
  // masked.
  auto store_tile = [&](int q) -> bool {
    const int t = t_begin + q / KT;
    const int m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;
    const int col = n0 + wn * 32 + l32;
    const bool full = m0 + BM <= M && n0 + BN <= N;
    if (full) {
      const float b = BIAS ? bias[col] : 0.0f;
      const int64_t base = (int64_t)(m0 + wm * 64 + half * 4) * N + col;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float v = acc[i][e];
          if (BIAS) v = v + b;
          store_out<OUT>(Y, base + (int64_t)(i * 32 + (e >> 2) * 8 + (e & 3)) * N, v);
        }
    } else if (col < N) {
      const float b = BIAS ? bias[col] : 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
          if (row < M) {
            float v = acc[i][e];
            if (BIAS) v = v + b;
            store_out<OUT>(Y, (int64_t)row * N + col, v);
          }
        }
    }
    acc[0] = (v16f){};
    acc[1] = (v16f){};
    return full;
  };
  auto store_partials = [&](int q, int gi, const v16i (&p)[2]) {
    const int t = t_begin + q / KT, g = (q % KT) * GPT + gi;
    const int m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;
    const int col = n0 + wn * 32 + l32;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
        if (row < M && col < N) partials[((int64_t)g * M + row) * N + col] = p[i][e];
      }
  };

  // One K step (half of a super-step); (pc, sc) receive this step's group, (pp, sp)
  // hold the previous one, whose VALU epilogue is interleaved with this step's MFMAs.
  auto half_step = [&](int q, v16i (&pc)[2], v16f (&sc)[2], v16i (&pp)[2], v16f (&sp)[2]) {
    const int kt = q % KT;
    const int slot = q % NSLOT;
    if (MODE == 1) {
#pragma unroll
      for (int gi = 0; gi < GPT; ++gi) {
        Frags f;
        load_frags(slot, gi, f);
        mfma_group(f, pc);
        store_partials(q, gi, pc);
      }
      return;
    }
    if constexpr (GPT == 1) {
      // sp is zero at a tile's first step, so the previous-group epilogue is unconditional
      Frags f;
      load_frags(slot, 0, f);
      mfma_group(f, pc);
      scale_group(f, sc);
      epilogue(pp, sp);
      __builtin_amdgcn_sched_group_barrier(0x100, 15, 0);  // DS reads: fragments + scales
#pragma unroll
      for (int m = 0; m < 8; ++m) {                         // 8 int8 MFMAs, VALU between
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
      }
#pragma unroll
      for (int m = 0; m < 2; ++m) {                         // 2 fp16 outer products
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
      }
      if (kt == KT - 1) {
        epilogue(pc, sc);
        store_tile(q);
        sc[0] = (v16f){};   // the next step (a new tile) adds cvt(pc) * 0
        sc[1] = (v16f){};
      }
    } else {
#pragma unroll
      for (int gi = 0; gi < GPT; ++gi) {
        Frags f;
        load_frags(slot, gi, f);
        mfma_group(f, pc);
        scale_group(f, sc);
        epilogue(pc, sc);
      }
      if (kt == KT - 1) store_tile(q);
    }
  };

  // Super-step: K steps q0 and q0+1 behind one barrier. Each wave first waits for all
  // of its outstanding vector-memory ops (the DMA of these two stages, issued one
  // super-step earlier, and any tile stores), then the barrier makes every wave's DMA
  // visible and guarantees the slots of the previous super-step are no longer read;
  // the next two stages are then prefetched into those slots.
  issue();
  if (total > 1) issue();
  v16i p0[2], p1[2];
  v16f s0[2], s1[2];
  p0[0] = p0[1] = p1[0] = p1[1] = (v16i){};
  s0[0] = s0[1] = s1[0] = s1[1] = (v16f){};
  for (int q = 0; q < total; q += 2) {
    KSD_WAIT_VM(0);
    wg_barrier();
    if (q + 2 < total) issue();
    if (q + 3 < total) issue();
    half_step(q, p0, s0, p1, s1);
    if (q + 1 < total) half_step(q + 1, p1, s1, p0, s0);
  }
}


// ---------------------------------------------------------------------------------------
// GS128 kernel (group == BK): one group per K step, eight 512-thread waves per CU.
//
//   * The same 128x128 tiles, tile order and 4-slot LDS ring as above, but each step's
//     DMA goes out as one scalar-based instruction per 1 KB (64-bit SGPR base + 32-bit
//     per-lane offset), and the LDS chunk swizzle XORs with (row >> 1) & 7: 16 consecutive
//     rows of one chunk column fill a 256-byte bank window (64 banks, no conflicts).
//   * Per wave and step: tile 0's four MFMAs and the fp16 scale outer product, under the
//     VALU epilogue of the previous step's tile 1; one barrier; tile 1's MFMAs, each
//     followed by the LDS reads of the next step's fragments for the k slice it just
//     consumed (the fragments double-buffer across steps), under this step's tile-0
//     epilogue. Tile 1's partial and scales wait in registers for the next step.
//   * A finished tile moves to a second accumulator and leaves in eight chunks of four
//     elements, one chunk per following step, through buffer stores whose descriptor
//     drops rows past M and columns past N. The output writes of all CUs are thus spread
//     over the next tile instead of bursting at every tile end.
//   * Waits: a wave's vector-memory loads complete in issue order, so "at most n
//     outstanding" (n = the instructions issued after step q+1's DMA) proves that DMA done;
//     pending stores only make such a wait stricter.
namespace g128 {
constexpr uint32_t SLOT = BM * BK;
// raw buffer resources: offsets at or past num_records drop stores
constexpr int kBufFlags = 0x00020000;
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ int swz16(int row, int chunk) {
  return row * BK + ((chunk ^ ((row >> 1) & 7)) << 4);
}
typedef __attribute__((address_space(3))) const v4i lds_v4i;
typedef __attribute__((address_space(3))) const uint32_t lds_u32;
__device__ __forceinline__ v4i lds16(uint32_t a) { return *(lds_v4i *)(uintptr_t)a; }
__device__ __forceinline__ uint32_t lds4(uint32_t a) { return *(lds_u32 *)(uintptr_t)a; }
// LDS DMA from base (SGPR pair) + off (per lane) into LDS at `lds` (wave-uniform)
__device__ __forceinline__ void dma16(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(off), "s"(base), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma2(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_ushort %0, %1" :: "v"(off), "s"(base), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void fenced_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  wg_barrier();
  __builtin_amdgcn_sched_barrier(0);
}
// s_waitcnt vmcnt(n) for the counts this kernel uses
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}
template <int OUT> __device__ __forceinline__ uint32_t out_bits(float v) {
  if constexpr (OUT == KSD_F32) return __builtin_bit_cast(uint32_t, v);
  else if constexpr (OUT == KSD_BF16) return f32_to_bf16(v);
  else if constexpr (OUT == KSD_F16) return f16_bits(v);
  else {  // KSD_F16_SAT: fp16, then clamp to +-65504
    _Float16 h = (_Float16)opaque(v);
    const float hf = (float)h;
    if (hf > kScaleMax) h = (_Float16)kScaleMax;
    if (hf < -kScaleMax) h = (_Float16)(-kScaleMax);
    return __builtin_bit_cast(uint16_t, h);
  }
}
struct Frags {
  v4i a[4][2], b[4];
  uint32_t sa[2], sw;
};

template <int OUT, bool BIAS>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_g128_kernel(
    const int8_t *__restrict__ A, const uint16_t *__restrict__ AS,
    const int8_t *__restrict__ W, const uint16_t *__restrict__ WS, int M, int N, int K,
    int tiles_n, int ntiles, const float *__restrict__ bias, void *__restrict__ Y) {
  __shared__ __attribute__((aligned(16))) int8_t sA[NSLOT][BM * BK];
  __shared__ __attribute__((aligned(16))) int8_t sW[NSLOT][BN * BK];
  __shared__ __attribute__((aligned(16))) uint32_t sS[NSLOT][256];
  constexpr int DEPTH = 3;  // steps of DMA in flight ahead of the step being computed
  constexpr int ES = OUT == KSD_F32 ? 4 : 2;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3, half = lane >> 5, l32 = lane & 31;
  const int G = K / BK, KT = K / BK;

  int t_begin, t_count;
  {
    const int nb = gridDim.x, per = nb / 8, rem = nb % 8, x = blockIdx.x % 8, i = blockIdx.x / 8;
    const int lb = x * per + min(x, rem) + i;
    t_begin = (int)((int64_t)ntiles * lb / nb);
    t_count = (int)((int64_t)ntiles * (lb + 1) / nb) - t_begin;
  }
  const int T = t_count * KT;
  if (T == 0) return;

  // ---- DMA: wave w fills A and W rows [16w, 16w+16) of a step (two 1 KB instructions
  // each); waves 0-3 also 64 scale rows (A [0,64), [64,128), W [0,64), [64,128)).
  const int drow0 = wave * 16 + (lane >> 3), drow1 = drow0 + 8;
  const int dch0 = ((lane & 7) ^ ((drow0 >> 1) & 7)) << 4;
  const int dch1 = ((lane & 7) ^ ((drow1 >> 1) & 7)) << 4;
  const bool s_load = wave < 4, s_isA = wave < 2;
  const int NW = s_load ? 5 : 4;  // vector-memory instructions per DMA step
  const int srow = (wave & 1) * 64 + lane;
  const uint32_t ldsA = lds_addr(&sA[0][0]) + wave * 2048;
  const uint32_t ldsW = lds_addr(&sW[0][0]) + wave * 2048;
  const uint32_t ldsS = lds_addr(&sS[0][0]) + ((s_isA ? 0 : 128) + (wave & 1) * 64) * 4;
  const uint16_t *const SB = s_isA ? AS : WS;
  const int8_t *ba, *bw;  // cursor: the next DMA step's tile bases (+ k) ...
  const uint16_t *bs;
  uint32_t oa0, oa1, ow0, ow1, os;  // ... and per-lane offsets (rows clamped into range)
  int cur_t = t_begin, cur_kt = 0;
  auto rebase = [&]() __attribute__((always_inline)) {
    const int m0 = (cur_t / tiles_n) * BM, n0 = (cur_t % tiles_n) * BN;
    ba = A + (int64_t)m0 * K;
    bw = W + (int64_t)n0 * K;
    const int r0 = s_isA ? m0 : n0, rmax = s_isA ? M : N;
    bs = SB + (int64_t)r0 * G;
    oa0 = (uint32_t)((min(m0 + drow0, M - 1) - m0) * K + dch0);
    oa1 = (uint32_t)((min(m0 + drow1, M - 1) - m0) * K + dch1);
    ow0 = (uint32_t)((min(n0 + drow0, N - 1) - n0) * K + dch0);
    ow1 = (uint32_t)((min(n0 + drow1, N - 1) - n0) * K + dch1);
    os = (uint32_t)((min(r0 + srow, rmax - 1) - r0) * G * 2);
  };
  rebase();
  auto dma_step = [&](uint32_t slot) __attribute__((always_inline)) {
    const uint32_t so = slot * SLOT;
    dma16(ba, oa0, ldsA + so);
    dma16(ba, oa1, ldsA + so + 1024);
    dma16(bw, ow0, ldsW + so);
    dma16(bw, ow1, ldsW + so + 1024);
    if (s_load) dma2(bs, os, ldsS + slot * 1024);
    ba += BK;
    bw += BK;
    bs += 1;
    if (++cur_kt == KT) {
      cur_kt = 0;
      if (++cur_t < t_begin + t_count) rebase();
    }
  };

  // ---- fragment addresses in slot 0 (slot s adds s * SLOT, or s * 1024 for scales)
  uint32_t adA[4][2], adB[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int kc = kk * 2 + half;
    adB[kk] = lds_addr(&sW[0][0]) + swz16(wn * 32 + l32, kc);
#pragma unroll
    for (int i = 0; i < 2; ++i) adA[kk][i] = lds_addr(&sA[0][0]) + swz16(wm * 64 + i * 32 + l32, kc);
  }
  const uint32_t adSa = lds_addr(&sS[0][0]) + (wm * 64 + l32) * 4;
  const uint32_t adSw = lds_addr(&sS[0][0]) + (128 + wn * 32 + l32) * 4;
  // lanes 32-63 supply k = 4..7 of the scale outer product: zeros
  const uint32_t smask = half ? 0u : 0xffffu;

  auto chain = [&](const Frags &f, int i) __attribute__((always_inline)) -> v16i {
    v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[0][i], f.b[0], (v16i){}, 0, 0, 0);
#pragma unroll
    for (int kk = 1; kk < 4; ++kk) p = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[kk][i], f.b[kk], p, 0, 0, 0);
    return p;
  };
  // sa (x) sw: an fp16 MFMA whose only non-zero k slot is 0, so every product is exact
  auto scale = [&](const Frags &f, int i) __attribute__((always_inline)) -> v16f {
    const v2u au = {f.sa[i] & smask, 0u}, bu = {f.sw & smask, 0u};
    return __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, au), __builtin_bit_cast(v4h, bu),
                                               (v16f){}, 0, 0, 0);
  };
  v16f acc[2], acc_old[2];
  acc[0] = acc[1] = acc_old[0] = acc_old[1] = (v16f){};
  auto ep = [&](int i, const v16i &p, const v16f &s) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = fmaf((float)p[e], s[e], acc[i][e]);
  };

  // ---- gradual store of the finished tile (acc_old): chunk c = elements 2c, 2c+1 of both
  // 32-row halves. Element e of a lane sits at row (e>>2)*8 + half*4 + (e&3) of its half.
  __amdgpu_buffer_rsrc_t ors0 = __builtin_amdgcn_make_buffer_rsrc(Y, 0, 0, kBufFlags), ors1 = ors0;
  int ovoff = 0, pend = 8;
  auto drain = [&](int c) __attribute__((always_inline)) {
    typedef uint32_t v16u __attribute__((ext_vector_type(16)));
    // (whole-vector bit casts: a bit cast of one vector element reads element 0 here)
    v16u o0, o1;
    if constexpr (OUT == KSD_F32) {
      o0 = __builtin_bit_cast(v16u, acc_old[0]);
      o1 = __builtin_bit_cast(v16u, acc_old[1]);
    }
#define KSD_DRAIN(C)                                                                      \
  case C:                                                                                 \
    _Pragma("unroll") for (int ee = 0; ee < 2; ++ee) {                                    \
      const int e = (C) * 2 + ee;                                                         \
      const int vo = ovoff + ((e >> 2) * 8 + (e & 3)) * N * ES;                           \
      if constexpr (OUT == KSD_F32) {                                                     \
        __builtin_amdgcn_raw_buffer_store_b32(o0[e], ors0, vo, 0, 0);                     \
        __builtin_amdgcn_raw_buffer_store_b32(o1[e], ors1, vo, 0, 0);                     \
      } else {                                                                            \
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)out_bits<OUT>(acc_old[0][e]), ors0, vo, 0, 0); \
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)out_bits<OUT>(acc_old[1][e]), ors1, vo, 0, 0); \
      }                                                                                   \
    }                                                                                     \
    break;
    switch (c) {
      KSD_DRAIN(0) KSD_DRAIN(1) KSD_DRAIN(2) KSD_DRAIN(3)
      KSD_DRAIN(4) KSD_DRAIN(5) KSD_DRAIN(6) KSD_DRAIN(7)
      default: break;
    }
#undef KSD_DRAIN
  };
  auto retire = [&](int t) __attribute__((always_inline)) {  // acc -> acc_old (tile t)
    while (pend < 8) drain(pend++);
    const int m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;
    const int col = n0 + wn * 32 + l32;
    const int64_t r0 = (int64_t)m0 + wm * 64;
    const int64_t rows0 = max((int64_t)0, min((int64_t)32, (int64_t)M - r0));
    const int64_t rows1 = max((int64_t)0, min((int64_t)32, (int64_t)M - r0 - 32));
    ors0 = __builtin_amdgcn_make_buffer_rsrc((char *)Y + r0 * N * ES, 0, (int)(rows0 * N * ES), kBufFlags);
    ors1 = __builtin_amdgcn_make_buffer_rsrc((char *)Y + (r0 + 32) * N * ES, 0, (int)(rows1 * N * ES), kBufFlags);
    ovoff = col < N ? (half * 4 * N + col) * ES : (int)kOob;
    const float b = BIAS ? (col < N ? bias[col] : 0.0f) : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_old[i][e] = BIAS ? acc[i][e] + b : acc[i][e];
    acc[0] = acc[1] = (v16f){};
    pend = 0;
  };

  const int pre = min(DEPTH, T);
  for (int i = 0; i < pre; ++i) dma_step((uint32_t)i);
  wait_vm((pre - 1) * NW);
  fenced_barrier();
  Frags F0, F1;
  {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      F0.b[kk] = lds16(adB[kk]);
      F0.a[kk][0] = lds16(adA[kk][0]);
      F0.a[kk][1] = lds16(adA[kk][1]);
    }
    F0.sa[0] = lds4(adSa);
    F0.sa[1] = lds4(adSa + 128);
    F0.sw = lds4(adSw);
  }
  v16i P1 = (v16i){};
  v16f S1 = (v16f){};
  int kt = 0, tk = t_begin;
  auto step = [&](int q, Frags &cur, Frags &nxt) __attribute__((always_inline)) {
    const v16i p0 = chain(cur, 0);
    const v16f s0 = scale(cur, 0);
    ep(1, P1, S1);  // tile 1 of step q-1 (zeros before the first step and after a retire)
#pragma unroll
    for (int m = 0; m < 5; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);  // VALU
    }
    // outstanding after step q+1's DMA: step q+2's (DMA issued in the previous step)
    if (q + 1 < T) wait_vm(q + 2 < T ? NW : 0);
    fenced_barrier();
    // step q+1's fragments, slice kk right after the tile-1 MFMA that last reads slice kk
    // of `cur` (at q = T-1 the reads hit a stale slot and are never used)
    const uint32_t ns = (uint32_t)((q + 1) & (NSLOT - 1));
    const uint32_t so = ns * SLOT, ss = ns * 1024;
    v16i p1 = (v16i){};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      p1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[kk][1], cur.b[kk], p1, 0, 0, 0);
      nxt.b[kk] = lds16(adB[kk] + so);
      nxt.a[kk][0] = lds16(adA[kk][0] + so);
      nxt.a[kk][1] = lds16(adA[kk][1] + so);
    }
    S1 = scale(cur, 1);
    nxt.sa[0] = lds4(adSa + ss);
    nxt.sa[1] = lds4(adSa + ss + 128);
    nxt.sw = lds4(adSw + ss);
    P1 = p1;
    ep(0, p0, s0);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
    if (++kt == KT) {
      ep(1, P1, S1);
      retire(tk);
      P1 = (v16i){};
      S1 = (v16f){};
      kt = 0;
      ++tk;
    } else if (pend < 8) {
      drain(pend++);
    }
    if (q + DEPTH < T) dma_step((uint32_t)((q + DEPTH) & (NSLOT - 1)));
  };
  for (int q = 0; q < T; q += 2) {
    step(q, F0, F1);
    if (q + 1 >= T) break;
    step(q + 1, F1, F0);
  }
  while (pend < 8) drain(pend++);
}
}  // namespace g128

// one workgroup per CU; the CU count is a device constant, cached per device
static int cu_count() {
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

template <int GROUP, int OUT, bool BIAS, int MODE>
static void launch(const int8_t *a, const uint16_t *as, const int8_t *w, const uint16_t *ws,
                   int M, int N, int K, const float *bias, void *y, int32_t *partials,
                   hipStream_t st) {
  const int tn = (N + BN - 1) / BN, tm = (M + BM - 1) / BM;
  const int ntiles = tm * tn;
  const int grid = min(ntiles, cu_count());
  if constexpr (GROUP == 128 && MODE == 0)
    g128::gemm_g128_kernel<OUT, BIAS><<<dim3(grid), dim3(NTHREADS), 0, st>>>(
        a, as, w, ws, M, N, K, tn, ntiles, bias, y);
  else
    gemm_nt_kernel<GROUP, OUT, BIAS, MODE><<<dim3(grid), dim3(NTHREADS), 0, st>>>(
        a, as, w, ws, M, N, K, tn, ntiles, bias, y, partials);
}

template <int GROUP, int OUT>
static void launch_b(const int8_t *a, const uint16_t *as, const int8_t *w, const uint16_t *ws,
                     int M, int N, int K, const float *bias, void *y, hipStream_t st) {
  if (bias) launch<GROUP, OUT, true, 0>(a, as, w, ws, M, N, K, bias, y, nullptr, st);
  else launch<GROUP, OUT, false, 0>(a, as, w, ws, M, N, K, bias, y, nullptr, st);
}

template <int GROUP>
static int launch_o(const int8_t *a, const uint16_t *as, const int8_t *w, const uint16_t *ws,
                    int M, int N, int K, const float *bias, void *y, int y_dtype,
                    hipStream_t st) {
  switch (y_dtype) {
    case KSD_F32: launch_b<GROUP, KSD_F32>(a, as, w, ws, M, N, K, bias, y, st); break;
    case KSD_BF16: launch_b<GROUP, KSD_BF16>(a, as, w, ws, M, N, K, bias, y, st); break;
    case KSD_F16: launch_b<GROUP, KSD_F16>(a, as, w, ws, M, N, K, bias, y, st); break;
    case KSD_F16_SAT: launch_b<GROUP, KSD_F16_SAT>(a, as, w, ws, M, N, K, bias, y, st); break;
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
    case 32: return launch_o<32>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
    case 64: return launch_o<64>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
    default: return launch_o<128>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
  }
}

extern "C" int ksd_w8a8_group_partials(const int8_t *a, const int8_t *w, int64_t M, int64_t N,
                                       int64_t K, int group, int32_t *partials,
                                       void *stream) {
  int rc = gemm_checks(a, w, M, N, K, group);
  if (rc != KSD_OK) return rc;
  if (M == 0 || N == 0 || K == 0) return KSD_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (group) {
    case 32: launch<32, KSD_F32, false, 1>(a, nullptr, w, nullptr, (int)M, (int)N, (int)K, nullptr, nullptr, partials, st); break;
    case 64: launch<64, KSD_F32, false, 1>(a, nullptr, w, nullptr, (int)M, (int)N, (int)K, nullptr, nullptr, partials, st); break;
    default: launch<128, KSD_F32, false, 1>(a, nullptr, w, nullptr, (int)M, (int)N, (int)K, nullptr, nullptr, partials, st); break;
  }
  return check_launch("w8a8_group_partials");
}
