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

#include <type_traits>

namespace ksd {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
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
//   * Every wave issues the same five DMA instructions per step: two 1 KB chunks of A,
//     two of W and one half-wave load of 32 scale rows.
//   * The step body is instantiated once per ring slot, so every LDS offset is an
//     immediate. Per wave and step: one barrier; the fp16 scale outer products of step
//     q-1 (two MFMAs, issued first so their results are ready when the epilogue needs
//     them); the DMA of step q+3; the fragment reads of step q; then step q's eight int8
//     MFMAs, each followed by 8 VALU of step q-1's epilogue (sched_group_barrier), so the
//     matrix pipe and the VALU run side by side. The partials ping-pong by step parity.
//   * The int32 chains start from the bits of 1.5*2^23 (12582912.0f) instead of zero:
//     |P_g| < 2^22 keeps C + P_g in one binade with unit ulp, so the partial's bits read as
//     an fp32 are exactly 12582912 + P_g and one exact v_sub_f32 gives float(P_g) (the
//     half-rate v_cvt_f32_i32 is not needed). The contract is unchanged:
//     acc = fmaf(float(P_g), sa*sw, acc).
//   * A finished tile is stored at once (32 buffer stores per lane) through descriptors
//     that drop rows past M and columns past N. Unit ends and DMA re-bases are marked
//     unlikely, so the hot loop stays compact.
//   * Waits: a wave's vector-memory operations complete in issue order, so "at most n
//     outstanding" (n = the instructions issued after step q's DMA) proves that DMA done;
//     the three steps after a unit end count its 32 stores into n.
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
    case 42: asm volatile("s_waitcnt vmcnt(42)" ::: "memory"); break;
    case 37: asm volatile("s_waitcnt vmcnt(37)" ::: "memory"); break;
    case 32: asm volatile("s_waitcnt vmcnt(32)" ::: "memory"); break;
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
// Cache policy of the output tile stores: nt (non-temporal, the gfx940+ meaning of the slc
// bit), so the streamed output does not evict the operand panels that other workgroups
// still read from L2 (config 3's forward: 1.92 -> 1.75 ms; config 2's step 0.154 -> 0.148 ms).
// K-part partials of a split launch keep the default policy: the combine kernel reads them
// right after (nt stores made config 5's combines 20% slower).
constexpr int kStoreNT = 2;
constexpr int kSeedBits = 0x4B400000;
constexpr float kSeedF = 12582912.0f;

// K-part p of `splits` covers steps [part_lo(p), part_lo(p + 1)) of the KT steps.
__host__ __device__ __forceinline__ int part_lo(int p, int KT, int splits) {
  return (int)((int64_t)p * KT / splits);
}

// One GEMM of a launch: Y (M, N) = A (M, K) . W (N, K)^T with its scales. Work unit u =
// (tile u / splits, K-part u % splits). With splits > 1, Y is the fp32 workspace: part p of
// a tile goes to Y + p * part_stride (elements), raw (no bias), and a combine kernel adds
// the parts in order. `out` is the output type (read by paired launches; single launches
// take it as a template argument).
struct G128Prob {
  const int8_t *A;
  const uint16_t *AS;
  const int8_t *W;
  const uint16_t *WS;
  const float *bias;
  void *Y;
  const void *R;
  int64_t part_stride;
  int M, N, K, tiles_n, ntiles, splits, out;
  // kOutSpine launches only: the per-chart increment table (N x 256 fp32) and the h
  // scales (M x tiles_n fp16); Y holds the h codes (M x N int8)
  const float *tab;
  uint16_t *hs;
};
// OUT of a launch whose epilogue is the KS3 spine, ReLU^2 and requantization (group 128)
// instead of a store of the accumulator.
constexpr int kOutSpine = 16;
// Work split of a paired launch over its grid (logical workgroup c, XCD-ordered): c takes
// q0 + (c < r0) consecutive units of problem 0 (the one with the longer units), then a run
// of problem 1's units, kA of them for c < r0 and kB for the others, so every workgroup
// ends near the same step count.
struct G128Sched {
  int q0, r0, kA, kB;
};
// Units of problem 1 before logical workgroup c (clamped to its unit count n1).
__device__ __forceinline__ int pair_start1(int c, const G128Sched &sc, int n1) {
  const int64_t s = c <= sc.r0 ? (int64_t)c * sc.kA : (int64_t)sc.r0 * sc.kA + (int64_t)(c - sc.r0) * sc.kB;
  return (int)(s < n1 ? s : n1);
}

// One stage of a max-butterfly over the 32 lanes of each half-wave: lanes with bit O of
// their index set keep values [O, 2O), the others [0, O), each maxed with the partner's
// copy (lane ^ O); after the stages O = 16 .. 1, lane l holds in r[0] the maximum over the
// half-wave of value index l.
template <int O>
__device__ __forceinline__ void bfly_max(uint32_t (&r)[32], int l32) {
  const bool up = (l32 & O) != 0;
#pragma unroll
  for (int k = 0; k < O; ++k) {
    const uint32_t send = up ? r[k] : r[k + O];
    const uint32_t keep = up ? r[k + O] : r[k];
    r[k] = max(keep, (uint32_t)__shfl_xor((int)send, O));
  }
}

// PAIR = false: one GEMM (p0; p1 is not read), output type OUT. PAIR = true: two
// independent GEMMs p0 and p1 in one persistent launch (no bias, no residual), each unit
// stored in its problem's runtime output type (OUT is ignored).
template <int OUT, bool BIAS, bool PAIR = false>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_g128_kernel(const G128Prob P0, const G128Prob P1,
                                                                const G128Sched sc) {
  __shared__ __attribute__((aligned(16))) int8_t sA[NSLOT][BM * BK];
  __shared__ __attribute__((aligned(16))) int8_t sW[NSLOT][BN * BK];
  __shared__ __attribute__((aligned(16))) uint32_t sS[NSLOT][256];
  // spine epilogue: [0, 512) per-wave row maxima (4 column waves x 128 rows), then per row
  // [512, 640) the ReLU^2 pre-scale or the h scale, [640, 768) its reciprocal
  __shared__ __attribute__((aligned(16))) uint32_t sRed[OUT == kOutSpine ? 768 : 4];
  constexpr int DEPTH = NSLOT - 1;
  constexpr int NW = 5;  // DMA instructions per wave and step: 4 x 1 KB codes + 1 scale

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3, half = lane >> 5, l32 = lane & 31;

  // This workgroup's work list: CU-local units v = 0 .. nbig-1 are problem 0's units
  // b_begin.., then (paired launches) v = nbig .. v_end-1 are problem 1's units s_begin..
  int b_begin, nbig, s_begin = 0, v_end;
  {
    const int nb = gridDim.x, per = nb / 8, rem = nb % 8, x = blockIdx.x % 8, i = blockIdx.x / 8;
    const int lb = x * per + min(x, rem) + i;
    if constexpr (!PAIR) {
      const int nunits = P0.ntiles * P0.splits;
      b_begin = (int)((int64_t)nunits * lb / nb);
      nbig = (int)((int64_t)nunits * (lb + 1) / nb) - b_begin;
      v_end = nbig;
    } else {
      b_begin = lb * sc.q0 + min(lb, sc.r0);
      nbig = sc.q0 + (lb < sc.r0 ? 1 : 0);
      const int n1 = P1.ntiles * P1.splits;
      s_begin = pair_start1(lb, sc, n1);
      v_end = nbig + pair_start1(lb + 1, sc, n1) - s_begin;
    }
  }
  // problem field of CU-local unit v (wave-uniform)
#define G128F(v, f) ((!PAIR || (v) < nbig) ? P0.f : P1.f)
  auto gunit = [&](int v) __attribute__((always_inline)) {
    return (!PAIR || v < nbig) ? b_begin + v : s_begin + (v - nbig);
  };
  auto unit_len = [&](int v) __attribute__((always_inline)) {
    const int sp = G128F(v, splits), KT = G128F(v, K) / BK, pp = gunit(v) % sp;
    return part_lo(pp + 1, KT, sp) - part_lo(pp, KT, sp);
  };
  int T = 0;
  if (!PAIR && P0.splits == 1) T = v_end * (P0.K / BK);
  else
    for (int v = 0; v < v_end; ++v) T += unit_len(v);
  if (T == 0) return;

  // DMA: each wave fills 16 rows of the A tile and 16 of the W tile (two 1 KB chunks of
  // each), and 32 rows of scales (A rows for waves 0-3, W rows for waves 4-7; lanes
  // 32-63 idle), so every wave issues the same 5 instructions per step.
  const int drow0 = wave * 16 + (lane >> 3), drow1 = drow0 + 8;
  const int dch0 = ((lane & 7) ^ ((drow0 >> 1) & 7)) << 4;
  const int dch1 = ((lane & 7) ^ ((drow1 >> 1) & 7)) << 4;
  const bool s_isA = wave < 4;
  const int srow = (wave & 3) * 32 + l32;
  const uint32_t ldsA = lds_addr(&sA[0][0]) + wave * 2048;
  const uint32_t ldsW = lds_addr(&sW[0][0]) + wave * 2048;
  const uint32_t ldsS = lds_addr(&sS[0][0]) + wave * 128;
  const int8_t *ba, *bw;
  const uint16_t *bs;
  uint32_t oa0, oa1, ow0, ow1, os;
  int is_u = 0, is_k = 0, is_len = __builtin_amdgcn_readfirstlane(unit_len(0));
  auto rebase = [&]() __attribute__((always_inline)) {
    // every value here is wave-uniform; readfirstlane keeps the DMA bases in SGPRs
    const int v = __builtin_amdgcn_readfirstlane(is_u);
    const int u = gunit(v), sp = G128F(v, splits), M = G128F(v, M), N = G128F(v, N), K = G128F(v, K);
    const int KT = K / BK, G = KT, tn = G128F(v, tiles_n);
    const int t = u / sp, k0 = __builtin_amdgcn_readfirstlane(part_lo(u % sp, KT, sp));
    const int m0 = (t / tn) * BM, n0 = (t % tn) * BN;
    ba = G128F(v, A) + (int64_t)m0 * K + (int64_t)k0 * BK;
    bw = G128F(v, W) + (int64_t)n0 * K + (int64_t)k0 * BK;
    const int r0 = s_isA ? m0 : n0, rmax = s_isA ? M : N;
    bs = (s_isA ? G128F(v, AS) : G128F(v, WS)) + (int64_t)r0 * G + k0;
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
    if (half == 0) dma2(bs, os, ldsS + slot * 1024);
    ba += BK;
    bw += BK;
    bs += 1;
    if (__builtin_expect(++is_k == is_len, 0)) {
      is_k = 0;
      if (++is_u < v_end) {
        is_len = __builtin_amdgcn_readfirstlane(unit_len(is_u));
        rebase();
      }
    }
  };

  // fragment addresses in slot 0
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
  const uint32_t smask = half ? 0u : 0xffffu;
  const v16i kSeed = (v16i){kSeedBits, kSeedBits, kSeedBits, kSeedBits, kSeedBits, kSeedBits,
                            kSeedBits, kSeedBits, kSeedBits, kSeedBits, kSeedBits, kSeedBits,
                            kSeedBits, kSeedBits, kSeedBits, kSeedBits};
  // keep the seed in VGPRs (the MFMA reads srcC from VGPRs)
  v16i seedv = kSeed;
  asm volatile("" : "+v"(seedv));
  v16f acc0 = (v16f){}, acc1 = (v16f){};
  int kt = 0, uk = 0, klen = is_len;

  auto store_impl = [&](auto out_c, int v) __attribute__((always_inline)) {
    constexpr int OT = decltype(out_c)::value;
    constexpr int ES = OT == KSD_F32 ? 4 : 2;
    const int u = gunit(v), sp = G128F(v, splits), tn = G128F(v, tiles_n);
    const int M = G128F(v, M), N = G128F(v, N);
    const float *const bias = G128F(v, bias);
    const void *const R = PAIR ? nullptr : P0.R;
    const int t = u / sp;
    char *const Yp = (char *)G128F(v, Y) + (int64_t)(u % sp) * G128F(v, part_stride) * ES;
    const int m0 = (t / tn) * BM, n0 = (t % tn) * BN;
    const int col = n0 + wn * 32 + l32;
    const int64_t r0 = (int64_t)m0 + wm * 64;
    const int64_t rows0 = max((int64_t)0, min((int64_t)32, (int64_t)M - r0));
    const int64_t rows1 = max((int64_t)0, min((int64_t)32, (int64_t)M - r0 - 32));
    __amdgpu_buffer_rsrc_t r0s = __builtin_amdgcn_make_buffer_rsrc(Yp + r0 * N * ES, 0, (int)(rows0 * N * ES), kBufFlags);
    __amdgpu_buffer_rsrc_t r1s = __builtin_amdgcn_make_buffer_rsrc(Yp + (r0 + 32) * N * ES, 0, (int)(rows1 * N * ES), kBufFlags);
    const int voff = col < N ? (half * 4 * N + col) * ES : (int)kOob;
    const float b = BIAS ? (col < N ? bias[col] : 0.0f) : 0.0f;
    // residual R (M, N) in the output type: y = out(out(acc + b) + r), the order of
    // `x + linear(...)` on tensors of the output dtype (one rounding per op)
    float r0v[16], r1v[16];
    if (R != nullptr) {
      __amdgpu_buffer_rsrc_t q0 = __builtin_amdgcn_make_buffer_rsrc((char *)R + r0 * N * ES, 0, (int)(rows0 * N * ES), kBufFlags);
      __amdgpu_buffer_rsrc_t q1 = __builtin_amdgcn_make_buffer_rsrc((char *)R + (r0 + 32) * N * ES, 0, (int)(rows1 * N * ES), kBufFlags);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int vo = voff + ((e >> 2) * 8 + (e & 3)) * N * ES;
        if constexpr (OT == KSD_F32) {
          r0v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(q0, vo, 0, 0));
          r1v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(q1, vo, 0, 0));
        } else if constexpr (OT == KSD_BF16) {
          r0v[e] = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(q0, vo, 0, 0) << 16);
          r1v[e] = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(q1, vo, 0, 0) << 16);
        } else {
          r0v[e] = (float)__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(q0, vo, 0, 0));
          r1v[e] = (float)__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(q1, vo, 0, 0));
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int vo = voff + ((e >> 2) * 8 + (e & 3)) * N * ES;
      float y0 = BIAS ? acc0[e] + b : acc0[e];
      float y1 = BIAS ? acc1[e] + b : acc1[e];
      if (R != nullptr) {
        if constexpr (OT == KSD_BF16) {
          y0 = __builtin_bit_cast(float, (uint32_t)f32_to_bf16(y0) << 16);
          y1 = __builtin_bit_cast(float, (uint32_t)f32_to_bf16(y1) << 16);
        } else if constexpr (OT != KSD_F32) {
          y0 = f16_round(y0);
          y1 = f16_round(y1);
        }
        y0 = y0 + r0v[e];
        y1 = y1 + r1v[e];
      }
      if constexpr (OT == KSD_F32) {
        if (sp > 1) {  // K-part partials: the combine kernel reads them next, from L2
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y0), r0s, vo, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y1), r1s, vo, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y0), r0s, vo, 0, kStoreNT);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y1), r1s, vo, 0, kStoreNT);
        }
      } else {
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)out_bits<OT>(y0), r0s, vo, 0, kStoreNT);
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)out_bits<OT>(y1), r1s, vo, 0, kStoreNT);
      }
    }
  };
  // The KS3 spine of the fused projection (ks3_triton.py:137-156, 'int8' mode) on the
  // finished tile: per element x = clamp(acc, +-65504), the chart's increment at the LUT
  // index of x / 4 (table gathered from global memory, L2-resident), h = x + inc; per row
  // the ReLU^2 pre-scale of max |h| over the tile's 128 charts (one GS128 group), codes
  // q = clamp(rint(h / pre), 0, 127), features (q * q) * (pre * pre); then the features'
  // own GS128 scale and int8 codes. The arithmetic is ks3_spine_fused_kernel's, element
  // for element. Row maxima: a butterfly over the 32 lanes of each half-wave leaves lane
  // l the maximum of its value index l (one row of the wave), the 4 column waves meet in
  // LDS, and 128 threads turn each row's maximum into its scale and reciprocal.
  auto spine_store = [&](int v) __attribute__((always_inline)) {
    if constexpr (OUT == kOutSpine) {
      const int t = gunit(v);  // one unit per tile (no K split)
      const int m0 = __builtin_amdgcn_readfirstlane((t / P0.tiles_n) * BM);
      const int n0 = __builtin_amdgcn_readfirstlane((t % P0.tiles_n) * BN);
      // N through an empty asm: the store offsets below are then formed here, at the unit
      // end, instead of being hoisted out of the K loop into 32 live registers
      int N = P0.N;
      asm volatile("" : "+s"(N));
      N = __builtin_amdgcn_readfirstlane(N);
      const int M = P0.M, tn = P0.tiles_n;
      const int cl = wn * 32 + l32;  // this lane's chart within the tile
      const bool cok = n0 + cl < N;
      const int ncol = min(N - n0, BN);
      const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(P0.tab + (int64_t)n0 * 256), 0, ncol * 1024, kBufFlags);
      float h[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const float a = k < 16 ? acc0[k] : acc1[k - 16];
        const float xc = fminf(fmaxf(a, -kScaleMax), kScaleMax);  // a NaN becomes -65504
        const int idx = min(max(lut_index_f32(xc * 0.25f) + 128, 0), 255);
        const float inc = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(trs, cok ? (uint32_t)(cl * 1024 + idx * 4) : kOob, 0, 0));
        h[k] = cok ? xc + inc : 0.0f;
      }
      // value index k of a lane: row wm*64 + (k >> 4)*32 + ((k & 15) >> 2)*8 + half*4 + (k & 3)
      const int krow = wm * 64 + (l32 >> 4) * 32 + ((l32 & 15) >> 2) * 8 + half * 4 + (l32 & 3);
      // per row of the tile: max over its 128 charts of the u32 patterns r (magnitudes, NaN
      // above inf), into sRed[512 + row] as the group scale and sRed[640 + row] as its
      // reciprocal; then the lane's 32 rows read back
      auto row_scales = [&](uint32_t (&r)[32], float (&sc)[32], float (&rc)[32]) __attribute__((always_inline)) {
        bfly_max<16>(r, l32);
        bfly_max<8>(r, l32);
        bfly_max<4>(r, l32);
        bfly_max<2>(r, l32);
        bfly_max<1>(r, l32);
        sRed[wn * 128 + krow] = r[0];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        fenced_barrier();
        if (tid < 128) {
          const uint32_t m = max(max(sRed[tid], sRed[128 + tid]), max(sRed[256 + tid], sRed[384 + tid]));
          const float s = group_scale(__builtin_bit_cast(float, m));
          sRed[512 + tid] = __builtin_bit_cast(uint32_t, s);
          sRed[640 + tid] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_rcpf(s));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        fenced_barrier();
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int row = wm * 64 + i * 32 + q * 8 + half * 4;
            // float vectors, read element by element (a __builtin_bit_cast of a vector
            // element reads element 0 whatever the index: hipcc 7.2, gfx950)
            const v4f s4 = *(const v4f *)&sRed[512 + row];
            const v4f r4 = *(const v4f *)&sRed[640 + row];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              sc[i * 16 + q * 4 + j] = s4[j];
              rc[i * 16 + q * 4 + j] = r4[j];
            }
          }
      };
      uint32_t r[32];
      float sc[32], rc[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) r[k] = __builtin_bit_cast(uint32_t, fabsf(h[k]));
      row_scales(r, sc, rc);
      // ReLU^2 codes and features (the pre-scale pre = sc)
      float tq[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const float p = h[k] * rc[k];
        tq[k] = rintf(p);
        if (fabsf(fabsf(p - tq[k]) - 0.5f) < 0x1p-14f) tq[k] = rintf(h[k] / sc[k]);
      }
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const float q = __builtin_amdgcn_fmed3f(tq[k], 0.0f, 127.0f);  // NaN q: NaN via pre
        h[k] = (q * q) * (sc[k] * sc[k]);
        r[k] = __builtin_bit_cast(uint32_t, fabsf(h[k]));
      }
      row_scales(r, sc, rc);
      // the features' codes (codes_rcp_packed, one value per row): rint(f / s) in [-127, 127]
      // through the reciprocal, the division near a half-integer, 0 for a NaN scale
      constexpr float kMagic = 12582912.0f;
      uint32_t code[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const float c = __builtin_amdgcn_fmed3f(h[k] * rc[k], -127.0f, 127.0f);
        const float m = c + kMagic;
        code[k] = __builtin_bit_cast(uint32_t, m);
        if (half_dist(c) < 0x1p-14f) code[k] = (uint8_t)code_of(h[k] / sc[k]);
      }
      // masked global stores: a buffer descriptor here would be held in VGPRs (the kernel's
      // SGPRs are full) and each store wrapped in a loop over its distinct values. The
      // table gathers above have returned before these stores issue (their values were
      // used), so every DMA issued before them is complete; the waits of the steps after
      // the unit end therefore hold whatever number of stores a wave issues here (masked
      // rows and charts may skip some).
      const int rows = max(0, min(BM, M - m0));
      int8_t *const qb = (int8_t *)P0.Y + (int64_t)m0 * N + n0 + cl;
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const int row = wm * 64 + (k >> 4) * 32 + ((k & 15) >> 2) * 8 + half * 4 + (k & 3);
        const uint32_t c = sc[k] != sc[k] ? 0u : code[k] & 0xffu;
        if (cok && row < rows) qb[(int64_t)row * N] = (int8_t)c;
      }
      if (tid < rows) {  // waves 0 and 1: row m0 + tid's scale of this group
        const float s = __builtin_bit_cast(float, sRed[512 + tid]);
        P0.hs[(int64_t)(m0 + tid) * tn + n0 / BN] = scale_bits(s);
      }
    }
  };
  auto store_tile = [&](int v) __attribute__((always_inline)) {
    if constexpr (OUT == kOutSpine) {
      spine_store(v);
    } else if constexpr (!PAIR) {
      store_impl(std::integral_constant<int, OUT>{}, v);
    } else {  // the unit's runtime output type (paired launches: fp32, bf16 or fp16)
      const int ot = G128F(v, out);
      if (ot == KSD_F32) store_impl(std::integral_constant<int, KSD_F32>{}, v);
      else if (ot == KSD_BF16) store_impl(std::integral_constant<int, KSD_BF16>{}, v);
      else store_impl(std::integral_constant<int, KSD_F16>{}, v);
    }
  };
  // acc += (P - seed) * S per element: the ordered contract for one group, P the seeded
  // int32 partials read as fp32, S the scale products
  auto epilogue = [&](const v16i &Q0, const v16i &Q1, const v16f &T0, const v16f &T1) __attribute__((always_inline)) {
    const v16f f0 = __builtin_bit_cast(v16f, Q0), f1 = __builtin_bit_cast(v16f, Q1);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      acc0[e] = fmaf(f0[e] - kSeedF, T0[e], acc0[e]);
      acc1[e] = fmaf(f1[e] - kSeedF, T1[e], acc1[e]);
    }
  };
  // sa (x) sw of a 32x32 tile from one f16 MFMA (k slot 0 only: lanes 32-63 hold zero);
  // the products of two fp16 values are exact in fp32
  auto scale_tile = [&](uint32_t sa, uint32_t sw) __attribute__((always_inline)) {
    const v2u a2 = {sa, 0u}, w2 = {sw, 0u};
    return __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, a2), __builtin_bit_cast(v4h, w2), (v16f){}, 0, 0, 0);
  };

  const int pre = min(DEPTH, T);
  for (int i = 0; i < pre; ++i) dma_step((uint32_t)i);

  // The epilogue of step q runs in step q+1, beside that step's MFMAs: partials ping-pong
  // by step parity, the scale bits wait in registers, and their products are formed at the
  // start of step q+1. Zero scales make the deferred epilogue a no-op (first step of a unit).
  v16i PA0 = seedv, PA1 = seedv, PB0 = seedv, PB1 = seedv;
  uint32_t qa0 = 0, qa1 = 0, qw = 0;
  int fresh = 0;  // steps left whose wait may leave the last unit's stores outstanding

  auto step = [&](auto slot_c, int q) __attribute__((always_inline)) {
    constexpr int S = decltype(slot_c)::value;
    constexpr uint32_t so = S * SLOT, ss = S * 1024;
    // This wave's DMA of step q has landed once at most the DMA of the (up to two) later
    // steps is outstanding. After a unit's 32 stores (issued after the DMA of the next three steps), the waits
    // of those three steps leave the stores outstanding: vector memory operations
    // complete in issue order, so "at most n + 32 outstanding" still proves this step's
    // DMA done.
    if (__builtin_expect(fresh == 0, 1)) {
      if (__builtin_expect(q + 2 < T, 1)) wait_vm(2 * NW);
      else if (q + 1 < T) wait_vm(NW);
      else wait_vm(0);
    } else {
      --fresh;
      if (q + 2 < T) wait_vm(2 * NW + 32);
      else if (q + 1 < T) wait_vm(NW + 32);
      else wait_vm(32);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    fenced_barrier();
    // the previous step's scale products first: the epilogue below needs them early
    const v16f T0 = scale_tile(qa0, qw), T1 = scale_tile(qa1, qw);
    asm volatile("" ::"v"(T0[0]), "v"(T1[0]));
    v16i &Pc0 = (S & 1) ? PB0 : PA0;
    v16i &Pc1 = (S & 1) ? PB1 : PA1;
    const v16i &Pp0 = (S & 1) ? PA0 : PB0;
    const v16i &Pp1 = (S & 1) ? PA1 : PB1;
    v4i b[4], a0[4], a1[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      b[kk] = lds16(adB[kk] + so);
      a0[kk] = lds16(adA[kk][0] + so);
      a1[kk] = lds16(adA[kk][1] + so);
    }
    const uint32_t sa0 = lds4(adSa + ss) & smask, sa1 = lds4(adSa + ss + 128) & smask, sw = lds4(adSw + ss) & smask;
    if (__builtin_expect(q + DEPTH < T, 1)) dma_step((uint32_t)((S + DEPTH) % NSLOT));
    v16i p0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0[0], b[0], seedv, 0, 0, 0);
    v16i p1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1[0], b[0], seedv, 0, 0, 0);
#pragma unroll
    for (int kk = 1; kk < 4; ++kk) {
      p0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0[kk], b[kk], p0, 0, 0, 0);
      p1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1[kk], b[kk], p1, 0, 0, 0);
    }
    epilogue(Pp0, Pp1, T0, T1);
    // issue order: fragment reads; the two scale MFMAs and the first int8 MFMA; then
    // 8 VALU of the previous step's epilogue per int8 MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 14, 0);  // 12 x b128 + 2 scale reads
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
    for (int j = 0; j < 7; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    Pc0 = p0;
    Pc1 = p1;
    qa0 = sa0;
    qa1 = sa1;
    qw = sw;
    if (__builtin_expect(++kt == klen, 0)) {  // unit end: fold in this step, store, restart
      const v16f U0 = scale_tile(qa0, qw), U1 = scale_tile(qa1, qw);
      epilogue(Pc0, Pc1, U0, U1);
      store_tile(uk);
      fresh = (PAIR || P0.R == nullptr) ? 3 : 0;
      acc0 = (v16f){};
      acc1 = (v16f){};
      qa0 = qa1 = qw = 0;
      kt = 0;
      if (++uk < v_end) klen = __builtin_amdgcn_readfirstlane(unit_len(uk));  // SGPR: scalar loop control
    }
  };
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, 2>;
  using C3 = std::integral_constant<int, 3>;
  // whole ring turns without exits, then the tail: an exit between the steps of the loop
  // body makes the compiler carry placeholder values for it through every step
  int q = 0;
  for (; q + NSLOT <= T; q += NSLOT) {
    step(C0{}, q);
    step(C1{}, q + 1);
    step(C2{}, q + 2);
    step(C3{}, q + 3);
  }
  if (q < T) {
    step(C0{}, q);
    if (q + 1 < T) {
      step(C1{}, q + 1);
      if (q + 2 < T) step(C2{}, q + 2);
    }
  }
}
// y = ((p_0 + p_1) + ...) + bias, then the output type: the parts of a split launch in
// ascending order, one fp32 rounding per add. 4 consecutive elements per thread.
template <int OUT, bool BIAS>
__global__ __launch_bounds__(256) void splitk_combine_kernel(const float *__restrict__ ws, int splits,
                                                            int64_t part_stride, int64_t n_elems, int N,
                                                            const float *__restrict__ bias,
                                                            void *__restrict__ Y, const void *__restrict__ R) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i0 >= n_elems) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = i0 + j;
    if (i >= n_elems) break;
    float y = ws[i];
    for (int pp = 1; pp < splits; ++pp) y = y + ws[(int64_t)pp * part_stride + i];
    if (BIAS) y = y + bias[i % N];
    if (R != nullptr) {
      if constexpr (OUT == KSD_F32) {
        y = y + ((const float *)R)[i];
      } else if constexpr (OUT == KSD_BF16) {
        y = __builtin_bit_cast(float, (uint32_t)f32_to_bf16(y) << 16) +
            __builtin_bit_cast(float, (uint32_t)((const uint16_t *)R)[i] << 16);
      } else {
        y = f16_round(y) + (float)__builtin_bit_cast(_Float16, ((const uint16_t *)R)[i]);
      }
    }
    if constexpr (OUT == KSD_F32) ((float *)Y)[i] = y;
    else ((uint16_t *)Y)[i] = (uint16_t)out_bits<OUT>(y);
  }
}
}  // namespace g128

// Split count of the GS128 GEMM for a shape: a launch with fewer than 192 output tiles of
// 128 x 128 splits K into up to 8 parts of at least 8 steps, aiming at 256 work units. It is
// a function of the shape only (the contract must not depend on the device).
static int g128_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN), KT = K / BK;
  if (tiles <= 0 || tiles >= 192) return 1;
  int64_t s = 256 / tiles;
  s = s < KT / 8 ? s : KT / 8;
  s = s < 8 ? s : 8;
  return s < 1 ? 1 : (int)s;
}


template <int GROUP, int OUT, bool BIAS, int MODE>
static void launch(const int8_t *a, const uint16_t *as, const int8_t *w, const uint16_t *ws,
                   int M, int N, int K, const float *bias, void *y, int32_t *partials,
                   hipStream_t st, int splits = 1, float *workspace = nullptr,
                   const void *residual = nullptr) {
  const int tn = (N + BN - 1) / BN, tm = (M + BM - 1) / BM;
  const int ntiles = tm * tn;
  if constexpr (GROUP == 128 && MODE == 0) {
    const g128::G128Sched none{0, 0, 0, 0};
    if (splits > 1) {
      const int64_t nel = (int64_t)M * N;
      const int grid = min(ntiles * splits, cu_count());
      const g128::G128Prob p{a, as, w, ws, nullptr, workspace, nullptr, nel, M, N, K, tn, ntiles, splits, KSD_F32};
      g128::gemm_g128_kernel<KSD_F32, false><<<dim3(grid), dim3(NTHREADS), 0, st>>>(p, p, none);
      const int64_t cb = (nel + 1023) / 1024;
      g128::splitk_combine_kernel<OUT, BIAS><<<dim3((unsigned)cb), dim3(256), 0, st>>>(
          workspace, splits, nel, nel, N, bias, y, residual);
    } else {
      const int grid = min(ntiles, cu_count());
      const g128::G128Prob p{a, as, w, ws, bias, y, residual, 0, M, N, K, tn, ntiles, 1, OUT};
      g128::gemm_g128_kernel<OUT, BIAS><<<dim3(grid), dim3(NTHREADS), 0, st>>>(p, p, none);
    }
  } else {
    const int grid = min(ntiles, cu_count());
    gemm_nt_kernel<GROUP, OUT, BIAS, MODE><<<dim3(grid), dim3(NTHREADS), 0, st>>>(
        a, as, w, ws, M, N, K, tn, ntiles, bias, y, partials);
  }
}

template <int GROUP, int OUT>
static void launch_b(const int8_t *a, const uint16_t *as, const int8_t *w, const uint16_t *ws,
                     int M, int N, int K, const float *bias, void *y, hipStream_t st,
                     int splits, float *workspace, const void *residual) {
  if (bias) launch<GROUP, OUT, true, 0>(a, as, w, ws, M, N, K, bias, y, nullptr, st, splits, workspace, residual);
  else launch<GROUP, OUT, false, 0>(a, as, w, ws, M, N, K, bias, y, nullptr, st, splits, workspace, residual);
}

template <int GROUP>
static int launch_o(const int8_t *a, const uint16_t *as, const int8_t *w, const uint16_t *ws,
                    int M, int N, int K, const float *bias, void *y, int y_dtype,
                    hipStream_t st, int splits = 1, float *workspace = nullptr,
                    const void *residual = nullptr) {
  switch (y_dtype) {
    case KSD_F32: launch_b<GROUP, KSD_F32>(a, as, w, ws, M, N, K, bias, y, st, splits, workspace, residual); break;
    case KSD_BF16: launch_b<GROUP, KSD_BF16>(a, as, w, ws, M, N, K, bias, y, st, splits, workspace, residual); break;
    case KSD_F16: launch_b<GROUP, KSD_F16>(a, as, w, ws, M, N, K, bias, y, st, splits, workspace, residual); break;
    case KSD_F16_SAT: launch_b<GROUP, KSD_F16_SAT>(a, as, w, ws, M, N, K, bias, y, st, splits, workspace, residual); break;
    default: return fail(KSD_ETYPE, "w8a8_gemm: unsupported output dtype %d", y_dtype);
  }
  return check_launch("w8a8_gemm_nt");
}

// Balanced work split of a paired launch (see G128Sched): problem 0 has n0 units of at
// most c0 steps each, problem 1 n1 units of at most c1 steps, c0 >= c1. The smallest
// per-workgroup step budget T that fits every unit gives kA / kB units of problem 1 to the
// workgroups with q0 + 1 / q0 units of problem 0.
static g128::G128Sched pair_sched(int64_t n0, int64_t c0, int64_t n1, int64_t c1, int grid) {
  g128::G128Sched sc{(int)(n0 / grid), (int)(n0 % grid), 0, 0};
  auto fill = [&](int64_t budget) { return budget < 0 ? (int64_t)0 : budget / c1; };
  const int64_t lo = (int64_t)(sc.q0 + (sc.r0 > 0 ? 1 : 0)) * c0;
  int64_t t = lo > (n0 * c0 + n1 * c1) / grid ? lo : (n0 * c0 + n1 * c1) / grid;
  for (;; ++t) {
    const int64_t a = fill(t - (int64_t)(sc.q0 + 1) * c0), b = fill(t - (int64_t)sc.q0 * c0);
    if (sc.r0 * a + (grid - sc.r0) * b >= n1) {
      sc.kA = (int)a;
      sc.kB = (int)b;
      return sc;
    }
  }
}

// Two GS128 GEMMs in one persistent launch: problem i is y_i (M_i, N_i) = a_i . w_i^T in
// output type dt_i (fp32, bf16 or fp16), with the same numeric contract (and K split) as
// its own launch. A problem whose shape splits K sums its parts in ws (fp32), then a
// combine kernel writes y_i.
static int launch_pair(const int8_t *const a[2], const uint16_t *const as[2], const int8_t *const w[2],
                       const uint16_t *const ws[2], const int64_t M[2], const int64_t N[2],
                       const int64_t K[2], void *const y[2], const int dt[2], float *workspace,
                       int64_t workspace_bytes, hipStream_t st) {
  g128::G128Prob p[2];
  int64_t cost[2], units[2], wsoff[2], need = 0;
  for (int i = 0; i < 2; ++i) {
    const int tn = (int)((N[i] + BN - 1) / BN), tm = (int)((M[i] + BM - 1) / BM);
    const int sp = g128_splits(M[i], N[i], K[i]);
    const int64_t KT = K[i] / BK;
    cost[i] = (KT + sp - 1) / sp;
    units[i] = (int64_t)tm * tn * sp;
    wsoff[i] = need;
    if (sp > 1) need += (int64_t)sp * M[i] * N[i] * 4;
    p[i] = g128::G128Prob{a[i], as[i], w[i], ws[i], nullptr, y[i], nullptr, 0, (int)M[i], (int)N[i],
                          (int)K[i], tn, tm * tn, sp, dt[i]};
  }
  if (need > 0 && (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 15) != 0))
    return fail(KSD_EINVAL, "w8a8_gemm_pair: needs a 16-byte aligned fp32 workspace of %lld bytes, "
                "got %lld", (long long)need, (long long)workspace_bytes);
  for (int i = 0; i < 2; ++i)
    if (p[i].splits > 1) {
      p[i].Y = (char *)workspace + wsoff[i];
      p[i].part_stride = M[i] * N[i];
      p[i].out = KSD_F32;
    }
  const int first = cost[1] > cost[0] ? 1 : 0;  // problem 0 of the launch: the longer units
  const g128::G128Prob &q0 = p[first], &q1 = p[1 - first];
  const int64_t n0 = units[first], n1 = units[1 - first];
  const int grid = (int)min((int64_t)cu_count(), n0 + n1);
  const g128::G128Sched sc = pair_sched(n0, cost[first], n1, cost[1 - first], grid);
  g128::gemm_g128_kernel<KSD_F32, false, true><<<dim3(grid), dim3(NTHREADS), 0, st>>>(q0, q1, sc);
  for (int i = 0; i < 2; ++i) {
    if (p[i].splits <= 1) continue;
    const int64_t nel = M[i] * N[i], cb = (nel + 1023) / 1024;
    const float *part = (const float *)((char *)workspace + wsoff[i]);
    switch (dt[i]) {
      case KSD_F32: g128::splitk_combine_kernel<KSD_F32, false><<<dim3((unsigned)cb), dim3(256), 0, st>>>(part, p[i].splits, nel, nel, (int)N[i], nullptr, y[i], nullptr); break;
      case KSD_BF16: g128::splitk_combine_kernel<KSD_BF16, false><<<dim3((unsigned)cb), dim3(256), 0, st>>>(part, p[i].splits, nel, nel, (int)N[i], nullptr, y[i], nullptr); break;
      default: g128::splitk_combine_kernel<KSD_F16, false><<<dim3((unsigned)cb), dim3(256), 0, st>>>(part, p[i].splits, nel, nel, (int)N[i], nullptr, y[i], nullptr); break;
    }
  }
  return check_launch("w8a8_gemm_pair");
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

extern "C" int ksd_w8a8_gemm_splits(int64_t M, int64_t N, int64_t K, int group, int *splits) {
  int rc = gemm_checks(reinterpret_cast<const int8_t *>(16), reinterpret_cast<const int8_t *>(16),
                       M, N, K, group);
  if (rc != KSD_OK) return rc;
  if (!splits) return fail(KSD_EINVAL, "w8a8_gemm_splits: null output");
  *splits = group == 128 ? g128_splits(M, N, K) : 1;
  return KSD_OK;
}

extern "C" int ksd_w8a8_gemm_nt_ex(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                                   const uint16_t *w_scales, int64_t M, int64_t N, int64_t K,
                                   int group, const float *bias, const void *residual, void *y,
                                   int y_dtype, float *workspace, int64_t workspace_bytes,
                                   void *stream) {
  int rc = gemm_checks(a, w, M, N, K, group);
  if (rc != KSD_OK) return rc;
  if (residual != nullptr) {
    if (group != 128) return fail(KSD_EINVAL, "w8a8_gemm: a residual needs group 128");
    if (y_dtype == KSD_F16_SAT) return fail(KSD_ETYPE, "w8a8_gemm: no residual with the saturating fp16 output");
  }
  if (M == 0 || N == 0) return KSD_OK;
  if (K == 0) return fail(KSD_EINVAL, "w8a8_gemm_nt_ex: K = 0 (the host wrapper handles it)");
  const int splits = group == 128 ? g128_splits(M, N, K) : 1;
  hipStream_t st = (hipStream_t)stream;
  if (splits > 1) {
    const int64_t need = (int64_t)splits * M * N * 4;
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 15) != 0)
      return fail(KSD_EINVAL, "w8a8_gemm: needs a 16-byte aligned fp32 workspace of %lld bytes "
                  "(%d K parts), got %lld", (long long)need, splits, (long long)workspace_bytes);
  }
  switch (group) {
    case 32: return launch_o<32>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
    case 64: return launch_o<64>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype, st);
    default: return launch_o<128>(a, a_scales, w, w_scales, (int)M, (int)N, (int)K, bias, y, y_dtype,
                                  st, splits, workspace, residual);
  }
}

extern "C" int ksd_w8a8_gemm_nt_ws(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                                   const uint16_t *w_scales, int64_t M, int64_t N, int64_t K,
                                   int group, const float *bias, void *y, int y_dtype,
                                   float *workspace, int64_t workspace_bytes, void *stream) {
  if (M == 0 || N == 0 || K == 0) return gemm_checks(a, w, M, N, K, group);
  return ksd_w8a8_gemm_nt_ex(a, a_scales, w, w_scales, M, N, K, group, bias, nullptr, y, y_dtype,
                             workspace, workspace_bytes, stream);
}

extern "C" int ksd_w8a8_gemm_pair(const int8_t *a0, const uint16_t *a0_scales, const int8_t *w0,
                                  const uint16_t *w0_scales, int64_t M0, int64_t N0, int64_t K0,
                                  void *y0, int y0_dtype, const int8_t *a1, const uint16_t *a1_scales,
                                  const int8_t *w1, const uint16_t *w1_scales, int64_t M1, int64_t N1,
                                  int64_t K1, void *y1, int y1_dtype, float *workspace,
                                  int64_t workspace_bytes, void *stream) {
  const int8_t *a[2] = {a0, a1}, *w[2] = {w0, w1};
  const uint16_t *as[2] = {a0_scales, a1_scales}, *ws[2] = {w0_scales, w1_scales};
  const int64_t M[2] = {M0, M1}, N[2] = {N0, N1}, K[2] = {K0, K1};
  void *y[2] = {y0, y1};
  const int dt[2] = {y0_dtype, y1_dtype};
  for (int i = 0; i < 2; ++i) {
    int rc = gemm_checks(a[i], w[i], M[i], N[i], K[i], 128);
    if (rc != KSD_OK) return rc;
    if (dt[i] != KSD_F32 && dt[i] != KSD_BF16 && dt[i] != KSD_F16)
      return fail(KSD_ETYPE, "w8a8_gemm_pair: output dtype %d (fp32, bf16 or fp16 only)", dt[i]);
    if (M[i] > 0 && N[i] > 0 && K[i] == 0)
      return fail(KSD_EINVAL, "w8a8_gemm_pair: K = 0 (the host wrapper handles it)");
  }
  const bool e0 = M0 == 0 || N0 == 0, e1 = M1 == 0 || N1 == 0;
  hipStream_t st = (hipStream_t)stream;
  if (e0 && e1) return KSD_OK;
  if (e0 || e1) {  // one empty problem: a single launch of the other
    const int i = e0 ? 1 : 0;
    return ksd_w8a8_gemm_nt_ex(a[i], as[i], w[i], ws[i], M[i], N[i], K[i], 128, nullptr, nullptr, y[i],
                               dt[i], workspace, workspace_bytes, stream);
  }
  return launch_pair(a, as, w, ws, M, N, K, y, dt, workspace, workspace_bytes, st);
}

extern "C" int ksd_ks3_project_fused(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                                     const uint16_t *w_scales, int64_t M, int64_t F, int64_t K,
                                     const int8_t *spine_codes, const uint16_t *spine_scale,
                                     const uint16_t *warp_scale, const uint16_t *warp_shift,
                                     const int8_t *tanh_lut, int group, int8_t *h_codes,
                                     uint16_t *h_scales, float *table, void *stream) {
  if (group != 128)
    return fail(KSD_EINVAL, "ks3_project_fused: group 128 only (groups 32 and 64: w8a8_gemm_nt, "
                "then ks3_spine_fused)");
  int rc = gemm_checks(a, w, M, F, K, group);
  if (rc != KSD_OK) return rc;
  if (!a_scales || !w_scales || !spine_codes || !spine_scale || !warp_scale || !warp_shift || !tanh_lut)
    return fail(KSD_EINVAL, "ks3_project_fused: null input pointer");
  if (!h_codes || !h_scales) return fail(KSD_EINVAL, "ks3_project_fused: null output pointer");
  if (!table || ((uintptr_t)table & 15) != 0)
    return fail(KSD_EINVAL, "ks3_project_fused: table workspace must be a 16-byte aligned buffer");
  if (((uintptr_t)tanh_lut & 3) != 0) return fail(KSD_EINVAL, "ks3_project_fused: tanh_lut must be 4-byte aligned");
  // code stores address a tile's 128 rows from one base with 32-bit offsets
  if (F > (1LL << 31) / BM) return fail(KSD_EINVAL, "ks3_project_fused: F too large");
  if (M == 0 || F == 0) return KSD_OK;
  if (K == 0) return fail(KSD_EINVAL, "ks3_project_fused: K = 0 (the host wrapper handles it)");
  hipStream_t st = (hipStream_t)stream;
  rc = ks3_fused_table(spine_codes, spine_scale, warp_scale, warp_shift, tanh_lut, F, table, st);
  if (rc != KSD_OK) return rc;
  const int tn = (int)((F + BN - 1) / BN), tm = (int)((M + BM - 1) / BM);
  const int grid = min(tm * tn, cu_count());
  const g128::G128Sched none{0, 0, 0, 0};
  const g128::G128Prob p{a, a_scales, w, w_scales, nullptr, h_codes, nullptr, 0, (int)M, (int)F, (int)K,
                         tn, tm * tn, 1, g128::kOutSpine, table, h_scales};
  g128::gemm_g128_kernel<g128::kOutSpine, false><<<dim3(grid), dim3(NTHREADS), 0, st>>>(p, p, none);
  return check_launch("ks3_project_fused");
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
