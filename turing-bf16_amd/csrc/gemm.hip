// Scaled GEMM on CDNA4 fp16 MFMA: y = bf16(acc * sa[m] * sb[n] + bias[n]) with
// acc[m, n] = sum_k a16[m, k] * b16[n, k] in fp32.
//
// a is either already fp16 (a16 with fp32 inverse row scales sa) or bf16 that is
// converted to fp16 with an exact per-row power of two 2^p[m] on its way from
// registers into LDS, sa = 2^-p[m] (the fused path, tbf16/csrc/gemm_sm75.cu:78-226).
// b is fp16 (prepare_weight's w16) with fp32 inverse row scales sb.
//
// Tiling (gfx950, 64-wide waves, 160 KB LDS):
//  - block tile BM (rows of a) x BN (rows of b), k tile BK (32 or 64); WM x WN
//    waves, each owning a (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks
//    (v_mfma_f32_32x32x16_f16: 16 fp32 accumulators per lane per block).
//  - operands staged global -> VGPR -> LDS with 16-byte buffer loads. LDS rows
//    are BK fp16 with the 16-byte chunk index XOR-swizzled, so the 32-row
//    fragment reads (ds_read_b128) and the row stores are bank-conflict free.
//  - PF register sets are in flight: each k tile's global loads are issued PF
//    compute phases before they are stored to LDS.
//  - the headline shape (config 9) uses BK = 64, so that every global load
//    instruction covers whole 128-byte row segments: half the L2 requests of
//    BK = 32, which measurably raises the clock the chip holds under this
//    kernel. Two LDS stages of 64 KB; fragments are read one 16-wide k step
//    ahead of the MFMAs and the last k step of each tile runs after the tile's
//    barrier, covering the latency of the next tile's first LDS reads. An
//    instruction-group schedule spreads each step's LDS reads, A conversions,
//    LDS writes and global loads between its MFMAs.
//  - config 0 (BK = 32, three LDS stages in a ring, the next tile's first
//    fragments read before the barrier) and the plain two-stage loop of the
//    smaller tiles remain selectable.
//  - the MFMA's first operand is the b fragment, the second the a fragment, so a
//    lane's 16 accumulators are four runs of 4 consecutive n for one m. The
//    epilogue applies the scales and bias in fp32 straight from the
//    accumulators, rounds once to bf16 and regroups lanes with three register
//    exchanges (v_permlane32_swap, v_permlane16_swap, a DPP row_ror:8), so each
//    store instruction writes whole 128-byte rows with no LDS round trip or
//    barrier (plain 8-byte stores from the accumulators were written back in
//    partial sectors).
//  - block ids are remapped so that each XCD (8 per chip, round-robin dispatch)
//    gets a contiguous range of tiles, grouped 8 a-tiles deep for L2 reuse.
// M <= 64 (decode) uses a separate skinny kernel that splits K across waves
// (see skinny_kernel below).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "abi_util.h"
#include "common.h"

using namespace tbf16;

namespace {

// Byte offset of 16-byte chunk `chunk` of row `row` in a [rows][BK] fp16 tile.
// BK = 64: 128-byte rows, chunk ^= (row / 2) % 8; BK = 32: 64-byte rows,
// chunk ^= (row / 4) % 4. Either way 16 lanes reading 16 consecutive rows at one
// logical chunk, or 8 (4) lanes writing one row, touch 64 distinct banks.
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  if constexpr (BK == 64) return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
  else return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}

template <int BM, int BN, int WM, int WN, int BK, int PF, int NS, bool A_BF16, bool KEVEN>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                           const int32_t* __restrict__ a_exp,
                                                           const float* __restrict__ a_sinv,
                                                           const uint16_t* __restrict__ B, int64_t ldb,
                                                           const float* __restrict__ b_sinv,
                                                           const uint16_t* __restrict__ bias,
                                                           uint16_t* __restrict__ C, int64_t ldc, int M, int N,
                                                           int K_all, float* __restrict__ part, int kt_per) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int CPR = BK / 8;  // 16-byte chunks per tile row
  constexpr int RP = NT / CPR;  // rows covered by one pass of 16-byte loads
  constexpr int AL = BM / RP, BL = BN / RP;
  static_assert(FM >= 1 && FN >= 1 && AL * RP == BM && BL * RP == BN, "bad tile");
  constexpr int RB = BK * 2;  // bytes per LDS tile row
  constexpr int STAGE = (BM + BN) * RB;
  constexpr int NSTG = NS == 5 ? 2 : NS >= 3 ? 3 : 2;  // LDS stages
  constexpr bool SCHED = NS == 4;
  // after the stages: the epilogue's factors for the tile, sa[BM] and sb[BN] (fp32)
  // and bias[BN] (bf16), written once before the first barrier
  constexpr int SMEM = NSTG * STAGE + (BM + BN) * 4 + BN * 2;
  static_assert(SMEM <= 160 * 1024, "LDS");
  __shared__ __align__(16) uint8_t smem[SMEM];
  float* const sa_l = reinterpret_cast<float*>(smem + NSTG * STAGE);
  float* const sb_l = sa_l + BM;
  uint16_t* const bias_l = reinterpret_cast<uint16_t*>(sb_l + BN);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- tile assignment: XCD-contiguous ranges, then grouped raster ----
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int bid = blockIdx.x;
  const int nblk = gridDim.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  constexpr int GM = 8;
  const int group = bid / (GM * tiles_n), first = group * GM, gsize = min(tiles_m - first, GM);
  const int within = bid % (GM * tiles_n);
  const int m0 = (first + within % gsize) * BM;
  const int n0 = (within / gsize) * BN;
  // split K (part != nullptr): block (x, y) sums k tiles [y kt_per, (y + 1) kt_per)
  // of its tile into fp32 partial sums part[y]; the reduction applies the epilogue
  const int ks = part ? (int)blockIdx.y : 0;
  const int kbase = ks * kt_per * BK;
  const int K = part ? min(K_all - kbase, kt_per * BK) : K_all;

  // the epilogue's factors (rows past M / columns past N get 0 and are not stored)
  for (int t = tid; t < BM; t += NT) {
    float s = 0.f;
    if (m0 + t < M) {
      if constexpr (A_BF16) s = ldexp1(-a_exp[m0 + t]);
      else s = a_sinv[m0 + t];
    }
    sa_l[t] = s;
  }
  for (int t = tid; t < BN; t += NT) {
    const bool ok = n0 + t < N;
    sb_l[t] = ok ? b_sinv[n0 + t] : 0.f;
    bias_l[t] = ok && bias ? bias[n0 + t] : (uint16_t)0;
  }

  // ---- global -> register staging through buffer loads ----
  // One buffer resource per operand tile (SGPRs), loop-invariant 32-bit row
  // offsets (VGPRs) and the k offset in an SGPR: no per-iteration address math
  // in vector registers, so in-flight loads of other register sets are never
  // waited for early. Rows past M (N) lie past the resource's end and load as
  // zeros; a K tail (K % BK != 0) is zeroed by a select, compiled in only when
  // KEVEN is false (a select on a loaded value makes the compiler wait for that
  // load on the spot, which serialises the register pipeline).
  const int lrow = tid / CPR, lch = tid % CPR;
  const BufRes arsrc =
      make_res(A + (int64_t)m0 * lda + kbase, min<int64_t>((int64_t)(M - m0) * lda * 2 - kbase * 2, 0x7fffffff));
  const BufRes brsrc =
      make_res(B + (int64_t)n0 * ldb + kbase, min<int64_t>((int64_t)(N - n0) * ldb * 2 - kbase * 2, 0x7fffffff));
  int aoff[AL], boff[BL];
  float as[AL];
#pragma unroll
  for (int i = 0; i < AL; ++i) {
    const int r = lrow + i * RP;
    aoff[i] = (r * (int)lda + lch * 8) * 2;
    if constexpr (A_BF16) as[i] = m0 + r < M ? pow2f(a_exp[m0 + r]) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < BL; ++i) boff[i] = ((lrow + i * RP) * (int)ldb + lch * 8) * 2;
  uint4 ra[PF][AL], rb[PF][BL];
  auto gload = [&](uint4(&va)[AL], uint4(&vb)[BL], int kt) {
    const int koff = kt * BK * 2;
    const bool kok = KEVEN || kt * BK + lch * 8 < K;
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const uint4 v = buf_load16(arsrc, aoff[i], koff);
      va[i] = kok ? v : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) {
      const uint4 v = buf_load16(brsrc, boff[i], koff);
      vb[i] = kok ? v : make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&](const uint4(&ra)[AL], const uint4(&rb)[BL], int stg) {
    uint8_t* sA = smem + stg * STAGE;
    uint8_t* sB = sA + BM * RB;
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      uint4 v = ra[i];
      if constexpr (A_BF16) v = cvt_bf16x8_f16x8(v, as[i]);
      *reinterpret_cast<uint4*>(sA + swz<BK>(lrow + i * RP, lch)) = v;
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) *reinterpret_cast<uint4*>(sB + swz<BK>(lrow + i * RP, lch)) = rb[i];
  };

  floatx16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int fr = lane & 31, fk = lane >> 5;
  auto compute = [&](int stg) {
    const uint8_t* sA = smem + stg * STAGE;
    const uint8_t* sB = sA + BM * RB;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int c = 2 * s + fk;
      half8 bf[FN], af[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) bf[i] = *reinterpret_cast<const half8*>(sB + swz<BK>(wn * TN + i * 32 + fr, c));
#pragma unroll
      for (int j = 0; j < FM; ++j) af[j] = *reinterpret_cast<const half8*>(sA + swz<BK>(wm * TM + j * 32 + fr, c));
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], acc[i][j], 0, 0, 0);
    }
  };

  const int KT = (K + BK - 1) / BK;
  if constexpr (NS == 2) {
    // LDS stage kt % 2 holds k tile kt; register set r holds the tile with index
    // congruent to r mod PF. At step kt the free set (kt % PF) starts loading tile
    // kt + PF, so each tile's loads have PF compute phases to land.
  #pragma unroll
    for (int p = 0; p < PF; ++p)
      if (p < KT) gload(ra[p], rb[p], p);
    lstore(ra[0], rb[0], 0);
    __syncthreads();
    int kt0 = 0;
    // Steady state: every step of the group issues its loads unconditionally, so
    // the compiler's wait counts can let the younger register sets stay in flight.
    for (; kt0 + 2 * PF - 1 < KT; kt0 += PF) {
  #pragma unroll
      for (int u = 0; u < PF; ++u) {
        gload(ra[u], rb[u], kt0 + u + PF);
        compute((kt0 + u) & 1);
        lstore(ra[(u + 1) % PF], rb[(u + 1) % PF], (kt0 + u + 1) & 1);
        __syncthreads();
      }
    }
    // Tail: the last < 2 * PF tiles, with guarded loads.
    for (; kt0 < KT; kt0 += PF) {
  #pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int kt = kt0 + u;
        if (kt < KT) {
          if (kt + PF < KT) gload(ra[u], rb[u], kt + PF);
          compute(kt & 1);
          if (kt + 1 < KT) lstore(ra[(u + 1) % PF], rb[(u + 1) % PF], (kt + 1) & 1);
          __syncthreads();
        }
      }
    }
  } else if constexpr (NS == 5) {
    // Two LDS stages of BK = 64 (whole 128-byte row segments per global load) and
    // the last k step of every tile deferred past the tile's barrier: after the
    // barrier a wave issues the LDS reads of the next tile's first step and then
    // the deferred step's MFMAs, whose fragments it read before the barrier, so the
    // read latency hides behind them. Tile kt + 1 is stored (A in step 0, B in
    // step 1) into the stage freed by the previous barrier and the loads of tile
    // kt + 1 + PF go out into the register set just emptied.
    constexpr int SUB = BK / 16;
    static_assert(SUB == 4, "deferred-step loop assumes four k steps per tile");
    half8 fb[2][FN], fa[2][FM];
    auto fread = [&](half8(&bf)[FN], half8(&af)[FM], int stg, int s) {
      const uint8_t* sA = smem + stg * STAGE;
      const uint8_t* sB = sA + BM * RB;
      const int c = 2 * s + fk;
#pragma unroll
      for (int i = 0; i < FN; ++i) bf[i] = *reinterpret_cast<const half8*>(sB + swz<BK>(wn * TN + i * 32 + fr, c));
#pragma unroll
      for (int j = 0; j < FM; ++j) af[j] = *reinterpret_cast<const half8*>(sA + swz<BK>(wm * TM + j * 32 + fr, c));
    };
    auto mma = [&](const half8(&bf)[FN], const half8(&af)[FM]) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], acc[i][j], 0, 0, 0);
    };
    // staging in three parts: A rows [0, AL/2) in step 0, [AL/2, AL) in step 1,
    // B in step 2 (part q covers register slots [lo, hi) of one operand)
    auto stage_part = [&](int q, const uint4(&va)[AL], const uint4(&vb)[BL], int stg) {
      uint8_t* sA = smem + stg * STAGE;
      uint8_t* sB = sA + BM * RB;
      if (q < 2) {
#pragma unroll
        for (int i = q * AL / 2; i < (q + 1) * AL / 2; ++i) {
          uint4 v = va[i];
          if constexpr (A_BF16) v = cvt_bf16x8_f16x8(v, as[i]);
          *reinterpret_cast<uint4*>(sA + swz<BK>(lrow + i * RP, lch)) = v;
        }
      } else {
#pragma unroll
        for (int i = 0; i < BL; ++i) *reinterpret_cast<uint4*>(sB + swz<BK>(lrow + i * RP, lch)) = vb[i];
      }
    };
    auto load_part = [&](int q, uint4(&va)[AL], uint4(&vb)[BL], int kt) {
      const int koff = kt * BK * 2;
      const bool kok = KEVEN || kt * BK + lch * 8 < K;
      if (q < 2) {
#pragma unroll
        for (int i = q * AL / 2; i < (q + 1) * AL / 2; ++i) {
          const uint4 v = buf_load16(arsrc, aoff[i], koff);
          va[i] = kok ? v : make_uint4(0, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int i = 0; i < BL; ++i) {
          const uint4 v = buf_load16(brsrc, boff[i], koff);
          vb[i] = kok ? v : make_uint4(0, 0, 0, 0);
        }
      }
    };
    constexpr int MF = FN * FM, RD = FN + FM;
    constexpr int VT = A_BF16 ? 10 * AL : 0;  // VALU ops of converting half of a thread's A slots
    // instruction groups of one k step: the next step's reads first (two per
    // MFMA), then each MFMA followed by its share of the staging work
    auto sched = [&](int part, bool store, bool load, bool reads) {
      const int n = part < 0 ? 0 : part == 0 ? AL / 2 : part == 1 ? AL - AL / 2 : BL;
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        if (reads && 2 * i < RD) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (VT && store && part >= 0 && part < 2) __builtin_amdgcn_sched_group_barrier(0x002, (VT + MF - 1) / MF, 0);
        if (store && i >= MF - n) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        if (load && i >= MF - n) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // one tile: the deferred step of tile kt - 1 (if any), steps 0 .. SUB - 2 of
    // tile kt, staging of tile kt + 1 from set v and loads of tile kt + 1 + PF
    auto tile = [&](int kt, int v, bool deferred, bool store, bool load) {
      const int stg = kt & 1;
      fread(fb[0], fa[0], stg, 0);
      if (deferred) {
        mma(fb[1], fa[1]);
        sched(-1, false, false, false);
      }
#pragma unroll
      for (int s = 0; s < SUB - 1; ++s) {
        fread(fb[(s + 1) & 1], fa[(s + 1) & 1], stg, s + 1);
        if (store) stage_part(s, ra[v], rb[v], stg ^ 1);
        if (load) load_part(s, ra[v], rb[v], kt + 1 + PF);
        mma(fb[s & 1], fa[s & 1]);
        sched(s, store, load, true);
      }
      __syncthreads();
    };
    // prologue: tile 0 stored, tiles 1 .. PF in flight (tile j in set j % PF)
#pragma unroll
    for (int q = 0; q < PF; ++q)
      if (q < KT) gload(ra[q], rb[q], q);
    lstore(ra[0], rb[0], 0);
    if (PF < KT) gload(ra[0], rb[0], PF);
    __syncthreads();
    int kt0 = 0;
    for (; kt0 + 1 + PF + PF - 1 < KT; kt0 += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) tile(kt0 + u, (u + 1) % PF, kt0 + u > 0, true, true);
    }
    for (; kt0 < KT; kt0 += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int kt = kt0 + u;
        if (kt < KT) tile(kt, (u + 1) % PF, kt > 0, kt + 1 < KT, kt + 1 + PF < KT);
      }
    }
    mma(fb[1], fa[1]);  // the last tile's deferred step
  } else {
    // Three LDS stages in a ring (tile kt in stage kt % 3) and fragments read one
    // 16-wide k step ahead of the MFMAs that use them, the next tile's first step
    // included: an MFMA never waits on the LDS read issued just before it. In step
    // kt a wave stores tile kt + 2 (stage (kt + 2) % 3 = (kt - 1) % 3, whose last
    // reads finished before the previous barrier) and starts the global loads of
    // tile kt + 2 + PF into the register set just emptied; one barrier per tile
    // publishes tile kt + 2 and retires the reads of stage kt % 3.
    constexpr int SUB = BK / 16;
    static_assert(SUB % 2 == 0, "fragment double buffer needs an even number of k steps");
    half8 fb[2][FN], fa[2][FM];
    auto fread = [&](half8(&bf)[FN], half8(&af)[FM], int stg, int s) {
      const uint8_t* sA = smem + stg * STAGE;
      const uint8_t* sB = sA + BM * RB;
      const int c = 2 * s + fk;
#pragma unroll
      for (int i = 0; i < FN; ++i) bf[i] = *reinterpret_cast<const half8*>(sB + swz<BK>(wn * TN + i * 32 + fr, c));
#pragma unroll
      for (int j = 0; j < FM; ++j) af[j] = *reinterpret_cast<const half8*>(sA + swz<BK>(wm * TM + j * 32 + fr, c));
    };
    auto mma = [&](const half8(&bf)[FN], const half8(&af)[FM]) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], acc[i][j], 0, 0, 0);
    };
    // one k tile; LOAD/STORE/NEXT say whether tile kt + 2 + PF is loaded, tile
    // kt + 2 stored and tile kt + 1's first fragments read (guarded in the tail)
    // Optional instruction-group schedule (NS == 4): each MFMA of a k step is
    // followed by its share of the step's LDS reads, A conversions, LDS writes and
    // global loads, so a wave keeps the matrix pipe fed while it does them.
    constexpr int MF = FN * FM, RD = FN + FM, WR = AL + BL, LD = AL + BL;
    constexpr int VT = A_BF16 ? 20 * AL : 0;  // VALU ops of one tile's A conversion
    auto sched = [&](bool staging) {
      if constexpr (SCHED) {
#pragma unroll
        for (int i = 0; i < MF; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          if (i < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
          if (staging) {
            if (VT) __builtin_amdgcn_sched_group_barrier(0x002, (VT + MF - 1) / MF, 0);  // VALU
            if (i >= MF - WR) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
            if (i >= MF - LD) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    auto tile = [&](int kt, int stg, int u, bool store, bool load, bool next) {
      const int stg1 = stg == 2 ? 0 : stg + 1, stg2 = stg1 == 2 ? 0 : stg1 + 1;
#pragma unroll
      for (int s = 0; s < SUB; ++s) {
        if (s + 1 < SUB) fread(fb[(s + 1) & 1], fa[(s + 1) & 1], stg, s + 1);
        else if (next) fread(fb[0], fa[0], stg1, 0);
        if (s == 0) {
          if (store) lstore(ra[u], rb[u], stg2);
          if (load) gload(ra[u], rb[u], kt + 2 + PF);
        }
        mma(fb[s & 1], fa[s & 1]);
        sched(s == 0);
      }
      __syncthreads();
    };
    // prologue: tiles 0 and 1 stored, tiles 2 .. PF + 1 in flight (set j % PF)
    static_assert(PF >= 2, "three-stage ring needs two register sets");
#pragma unroll
    for (int q = 0; q < PF; ++q)
      if (q < KT) gload(ra[q], rb[q], q);
    lstore(ra[0], rb[0], 0);
    if (PF < KT) gload(ra[0], rb[0], PF);
    if (KT > 1) lstore(ra[1], rb[1], 1);
    if (PF + 1 < KT) gload(ra[1], rb[1], PF + 1);
    __syncthreads();
    fread(fb[0], fa[0], 0, 0);
    int kt0 = 0, stg = 0;
    for (; kt0 + 2 + PF + PF - 1 < KT; kt0 += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        tile(kt0 + u, stg, (u + 2) % PF, true, true, true);
        stg = stg == 2 ? 0 : stg + 1;
      }
    }
    for (; kt0 < KT; kt0 += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int kt = kt0 + u;
        if (kt < KT) {
          tile(kt, stg, (u + 2) % PF, kt + 2 < KT, kt + 2 + PF < KT, kt + 1 < KT);
          stg = stg == 2 ? 0 : stg + 1;
        }
      }
    }
  }

  // ---- epilogue: (acc * sa[m]) * sb[n] + bias[n] -> bf16 straight from registers ----
  // Lane l holds columns 8 q + 4 (l / 32) .. + 3 of row l % 32 for q = 0..3.
  // Exchanges regroup them without LDS or a barrier: v_permlane32_swap pairs q = 2p
  // (kept by lanes < 32) with q = 2p + 1 (kept by lanes >= 32), so a lane holds 8
  // columns (16 bytes) of its row; v_permlane16_swap then pairs p = 0 with p = 1
  // between 16-lane rows (lane l: row l % 16, or + 16, columns 0 / 16 / 8 / 24 of
  // the 32-column block for l / 16 = 0 / 1 / 2 / 3); where FN is even, a DPP
  // row_ror:8 exchange between lanes l and l ^ 8 then pairs blocks i - 1 and i, so
  // each store instruction writes whole 128-byte rows (8 rows x 64 columns) and L2
  // writes back exactly y (WRITE_SIZE = y; 64-byte runs had read 1.38 x).
  if (part) {
    // raw fp32 sums: acc[i][j][4 q + r] is row wm TM + 32 j + fr, column
    // wn TN + 32 i + 8 q + 4 fk + r of the tile (N is a multiple of 8)
    float* const pk = part + (int64_t)ks * M * N;
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int m = m0 + wm * TM + j * 32 + fr;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + wn * TN + i * 32 + 8 * q + 4 * fk;
          if (m < M && n < N)
            *reinterpret_cast<float4*>(pk + (int64_t)m * N + n) =
                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
        }
    }
    return;
  }
  const int rl = lane & 15, cq = lane >> 4;
  const int cl = ((cq & 1) << 4) | ((cq >> 1) << 3);
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int ml = wm * TM + j * 32 + fr;  // this lane's row before the exchanges
    const float sa = sa_l[ml];
    const int r0 = m0 + wm * TM + j * 32 + rl;  // rows stored by this lane
    uint32_t xa[4], ya[4];  // block i - 1's x / y, held for the third exchange
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      uint32_t w[4][2];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = wn * TN + i * 32 + 8 * q + 4 * fk;
        const float4 sb = *reinterpret_cast<const float4*>(sb_l + nl);
        const uint2 bw = *reinterpret_cast<const uint2*>(bias_l + nl);
        const float y0 = fmaf(acc[i][j][4 * q + 0] * sa, sb.x, bf16_lo(bw.x));
        const float y1 = fmaf(acc[i][j][4 * q + 1] * sa, sb.y, bf16_hi(bw.x));
        const float y2 = fmaf(acc[i][j][4 * q + 2] * sa, sb.z, bf16_lo(bw.y));
        const float y3 = fmaf(acc[i][j][4 * q + 3] * sa, sb.w, bf16_hi(bw.y));
        w[q][0] = pack_bf16(y0, y1);
        w[q][1] = pack_bf16(y2, y3);
      }
      // v[p]: 16 bytes of row l % 32, columns 16 p + 8 (l / 32) .. + 7
      uint32_t v[2][4];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const auto d0 = __builtin_amdgcn_permlane32_swap(w[2 * p][0], w[2 * p + 1][0], false, false);
        const auto d1 = __builtin_amdgcn_permlane32_swap(w[2 * p][1], w[2 * p + 1][1], false, false);
        v[p][0] = d0[0]; v[p][1] = d1[0]; v[p][2] = d0[1]; v[p][3] = d1[1];
      }
      // x: rows 0..15 of the 32-row block, y: rows 16..31
      uint32_t x[4], y[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const auto e = __builtin_amdgcn_permlane16_swap(v[0][d], v[1][d], false, false);
        x[d] = e[0];
        y[d] = e[1];
      }
      if constexpr (FN % 2 == 0) {
        if (i % 2 == 0) {
#pragma unroll
          for (int d = 0; d < 4; ++d) { xa[d] = x[d]; ya[d] = y[d]; }
          continue;
        }
        // third exchange: lane l and lane l ^ 8 (DPP row_ror:8) trade so that one
        // store writes rows 0..7 (or 8..15) with blocks i - 1 and i side by side
        const bool hi8 = (lane & 8) != 0;
        uint32_t f[4], s2[4], g[4], s3[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t tx = __builtin_amdgcn_mov_dpp((int)xa[d], 0x128, 0xF, 0xF, false);
          const uint32_t tb = __builtin_amdgcn_mov_dpp((int)x[d], 0x128, 0xF, 0xF, false);
          f[d] = hi8 ? tb : xa[d];
          s2[d] = hi8 ? x[d] : tx;
          const uint32_t uy = __builtin_amdgcn_mov_dpp((int)ya[d], 0x128, 0xF, 0xF, false);
          const uint32_t ub = __builtin_amdgcn_mov_dpp((int)y[d], 0x128, 0xF, 0xF, false);
          g[d] = hi8 ? ub : ya[d];
          s3[d] = hi8 ? y[d] : uy;
        }
        const int rb = m0 + wm * TM + j * 32 + (lane & 7);
        const int n = n0 + wn * TN + (i - 1 + (hi8 ? 1 : 0)) * 32 + cl;
        if (n < N) {
          if (rb < M) stg16(C + (int64_t)rb * ldc + n, make_uint4(f[0], f[1], f[2], f[3]));
          if (rb + 8 < M) stg16(C + (int64_t)(rb + 8) * ldc + n, make_uint4(s2[0], s2[1], s2[2], s2[3]));
          if (rb + 16 < M) stg16(C + (int64_t)(rb + 16) * ldc + n, make_uint4(g[0], g[1], g[2], g[3]));
          if (rb + 24 < M) stg16(C + (int64_t)(rb + 24) * ldc + n, make_uint4(s3[0], s3[1], s3[2], s3[3]));
        }
      } else {
        const int n = n0 + wn * TN + i * 32 + cl;
        if (n < N) {
          if (r0 < M) stg16(C + (int64_t)r0 * ldc + n, make_uint4(x[0], x[1], x[2], x[3]));
          if (r0 + 16 < M) stg16(C + (int64_t)(r0 + 16) * ldc + n, make_uint4(y[0], y[1], y[2], y[3]));
        }
      }
    }
  }
}

// Split-K reduction and epilogue: y = bf16((p_0 + p_1 + ...) * sa[m] * sb[n] +
// bias[n]) over the fp32 partial sums of gemm_kernel's split blocks, summed in
// split order (deterministic), with the same fp32 epilogue arithmetic as the
// unsplit kernel. One thread per 8 consecutive columns of a row; splits >= 2.
template <bool A_BF16>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                                            const int32_t* __restrict__ a_exp,
                                                            const float* __restrict__ a_sinv,
                                                            const float* __restrict__ b_sinv,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ C, int64_t ldc, int M, int N) {
  const int ng = N >> 3;
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= (int64_t)M * ng) return;
  const int m = (int)(g / ng), n = (int)(g % ng) * 8;
  const float* src = part + (int64_t)m * N + n;
  const int64_t stride = (int64_t)M * N;
  // split 1's loads go out with split 0's (no round trip between them)
  float4 lo = *reinterpret_cast<const float4*>(src), hi = *reinterpret_cast<const float4*>(src + 4);
  const float4 a1 = *reinterpret_cast<const float4*>(src + stride), b1 = *reinterpret_cast<const float4*>(src + stride + 4);
  lo.x += a1.x; lo.y += a1.y; lo.z += a1.z; lo.w += a1.w;
  hi.x += b1.x; hi.y += b1.y; hi.z += b1.z; hi.w += b1.w;
  for (int k = 2; k < splits; ++k) {
    const float* q = src + k * stride;
    const float4 a = *reinterpret_cast<const float4*>(q), b = *reinterpret_cast<const float4*>(q + 4);
    lo.x += a.x; lo.y += a.y; lo.z += a.z; lo.w += a.w;
    hi.x += b.x; hi.y += b.y; hi.z += b.z; hi.w += b.w;
  }
  float sa;
  if constexpr (A_BF16) sa = ldexp1(-a_exp[m]);
  else sa = a_sinv[m];
  const float4 s0 = *reinterpret_cast<const float4*>(b_sinv + n), s1 = *reinterpret_cast<const float4*>(b_sinv + n + 4);
  uint4 bw = make_uint4(0, 0, 0, 0);
  if (bias) bw = make_uint4(*reinterpret_cast<const uint32_t*>(bias + n), *reinterpret_cast<const uint32_t*>(bias + n + 2),
                            *reinterpret_cast<const uint32_t*>(bias + n + 4), *reinterpret_cast<const uint32_t*>(bias + n + 6));
  const uint4 out = make_uint4(pack_bf16(fmaf(lo.x * sa, s0.x, bf16_lo(bw.x)), fmaf(lo.y * sa, s0.y, bf16_hi(bw.x))),
                               pack_bf16(fmaf(lo.z * sa, s0.z, bf16_lo(bw.y)), fmaf(lo.w * sa, s0.w, bf16_hi(bw.y))),
                               pack_bf16(fmaf(hi.x * sa, s1.x, bf16_lo(bw.z)), fmaf(hi.y * sa, s1.y, bf16_hi(bw.z))),
                               pack_bf16(fmaf(hi.z * sa, s1.z, bf16_lo(bw.w)), fmaf(hi.w * sa, s1.w, bf16_hi(bw.w))));
  stg16(C + (int64_t)m * ldc + n, out);
}

// Skinny GEMM for M <= 32 * MB rows of a (decode and small batches). One block
// per 32 * NB rows of b; its NW waves split K into interleaved 64-wide chunks
// (wave w takes chunks w, w + NW, ...). Each operand value is used by a single
// wave, so both go global -> registers -> MFMA with no LDS staging: a lane loads
// 64 contiguous bytes of one row per chunk, and lane half h of MFMA k step j
// holds k = 32 h + 8 j + [0, 8) of the chunk for both operands (the same k-slot
// assignment on both sides gives the same dot products). PF chunks per wave are
// in flight. The NW partial tiles are summed through LDS in the epilogue and
// rounded once to bf16.
template <int NB, int MB, int NW, int PF, bool TR, bool A_BF16>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                         const int32_t* __restrict__ a_exp,
                                                         const float* __restrict__ a_sinv,
                                                         const uint16_t* __restrict__ B, int64_t ldb,
                                                         const float* __restrict__ b_sinv,
                                                         const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
                                                         int64_t ldc, int M, int N, int K, int R) {
  constexpr int NT = NW * 64, NBLK = NB * MB;
  constexpr int RED = NW * NBLK * 16 * 64 * 4, TSLOT = NB * 32 * 128;  // TR: one chunk of b rows per wave
  constexpr int SMEM = TR && NW * TSLOT > RED ? NW * TSLOT : RED;
  __shared__ __align__(16) uint8_t smem[SMEM];
  float* red = reinterpret_cast<float*>(smem);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, fh = lane >> 5;
  // block b owns weight rows [b R, b R + R), R <= 32 NB (a multiple of 4): R below
  // 32 NB spreads N over more blocks (one round over every CU) at the price of
  // zero rows in the MFMA tiles, which the memory-bound decode does not notice
  const int n0 = blockIdx.x * R;
  const int nend = min(N, n0 + R);
  uint8_t* tslot = smem + wave * TSLOT;

  // rows past N (M) lie past the resources' ends and load as zeros; pieces past
  // K are zeroed by a select
  const BufRes bres = make_res(B + (int64_t)n0 * ldb, min<int64_t>((int64_t)(nend - n0) * ldb * 2, 0x7fffffff));
  const BufRes ares = make_res(A, min<int64_t>((int64_t)M * lda * 2, 0x7fffffff));
  int boff[NB], aoff[MB];
  float as[MB];
  // TR: b is loaded coalesced (load q of block nb: rows 32 nb + 8 q + lane / 8,
  // 16-byte chunk lane % 8 of the chunk's 128-byte row piece) and transposed
  // into MFMA fragments through a per-wave LDS slot, the chunk index
  // XOR-swizzled by (row / 2) % 8 so that both sides are bank-conflict free.
  // Otherwise lane (r, h) loads 64 contiguous bytes of row r directly.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) boff[nb] = ((32 * nb + fr) * (int)ldb + 32 * fh) * 2;
  int toff[NB][4];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int q = 0; q < 4; ++q) toff[nb][q] = ((32 * nb + 8 * q + (lane >> 3)) * (int)ldb + 8 * (lane & 7)) * 2;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 32 * mb + fr;
    aoff[mb] = (m * (int)lda + 32 * fh) * 2;
    if constexpr (A_BF16) as[mb] = m < M ? pow2f(a_exp[m]) : 0.f;
  }
  const int KC = (K + 63) / 64;
  const int NI = wave < KC ? (KC - 1 - wave) / NW + 1 : 0;  // chunks of this wave

  uint4 wr[PF][NB][4], xr[PF][MB][4];
  // chunk i of this wave into a register set; only a wave's last chunk can run
  // past K, so the steady state loads without the zeroing select (a select
  // right after the load makes the compiler wait for the load there)
  auto gload = [&](uint4(&w)[NB][4], uint4(&x)[MB][4], int i, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int c = wave + i * NW;
    const int soff = c * 128;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool ok = !MASKED || c * 64 + 32 * fh + 8 * q < K;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if constexpr (TR) {
          // zero pieces past K (the piece's k is 8 * (lane % 8) of the chunk)
          const uint4 v = buf_load16(bres, toff[nb][q], soff);
          w[nb][q] = !MASKED || c * 64 + 8 * (lane & 7) < K ? v : make_uint4(0, 0, 0, 0);
        } else {
          const uint4 v = buf_load16(bres, boff[nb] + 16 * q, soff);
          w[nb][q] = ok ? v : make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint4 v = buf_load16(ares, aoff[mb] + 16 * q, soff);
        x[mb][q] = ok ? v : make_uint4(0, 0, 0, 0);
      }
    }
  };
  floatx16 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nb][mb][r] = 0.f;
  auto compute = [&](const uint4(&w)[NB][4], const uint4(&x)[MB][4]) {
    uint4 wt[NB][4];
    if constexpr (TR) {
      // through LDS: same wave, so program order keeps the previous chunk's reads
      // ahead of these writes
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = 32 * nb + 8 * q + (lane >> 3);
          *reinterpret_cast<uint4*>(tslot + row * 128 + (((lane & 7) ^ ((row >> 1) & 7)) << 4)) = w[nb][q];
        }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = 32 * nb + fr;
          wt[nb][j] = *reinterpret_cast<const uint4*>(tslot + row * 128 + (((4 * fh + j) ^ ((row >> 1) & 7)) << 4));
        }
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) wt[nb][j] = w[nb][j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half8 xf[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        xf[mb] = __builtin_bit_cast(half8, A_BF16 ? cvt_bf16x8_f16x8(x[mb][j], as[mb]) : x[mb][j]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[nb][mb] =
              __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, wt[nb][j]), xf[mb], acc[nb][mb], 0, 0, 0);
    }
  };
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (u < NI) gload(wr[u], xr[u], u, std::true_type{});
  int i0 = 0;
  // Steady state: unconditional loads, and scheduling barriers between the
  // steps so that the compiler keeps each step's loads after its MFMAs (left
  // free, it hoists the next chunks' loads, reuses their registers early and
  // ends up waiting for loads it has just issued). It loads chunks up to
  // i0 + 2 PF - 1 and stops before reaching the wave's last chunk NI - 1, the
  // only one that can run past K: that one is always loaded masked, below.
  for (; i0 + 2 * PF < NI; i0 += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      compute(wr[u], xr[u]);
      __builtin_amdgcn_sched_barrier(0);
      gload(wr[u], xr[u], i0 + u + PF, std::false_type{});
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  for (; i0 < NI; i0 += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      if (i0 + u < NI) {
        compute(wr[u], xr[u]);
        if (i0 + u + PF < NI) gload(wr[u], xr[u], i0 + u + PF, std::true_type{});
      }
    }
  }

  // ---- sum the NW partial tiles, scale, round once to bf16 ----
  if constexpr (TR) __syncthreads();  // the transpose slots alias red
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((wave * NBLK + nb * MB + mb) * 16 + r) * 64 + lane] = acc[nb][mb][r];
  __syncthreads();
  for (int g = tid; g < NBLK * 4 * 64; g += NT) {
    const int blk = g >> 8, rq = (g >> 6) & 3, ln = g & 63;
    const int nb = blk / MB, mb = blk % MB;
    const int m = 32 * mb + (ln & 31), n = n0 + 32 * nb + 8 * rq + 4 * (ln >> 5);
    if (m >= M || n >= nend) continue;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += red[((w * NBLK + blk) * 16 + 4 * rq + e) * 64 + ln];
    float sa;
    if constexpr (A_BF16) sa = ldexp1(-a_exp[m]);
    else sa = a_sinv[m];
    const float4 sb = *reinterpret_cast<const float4*>(b_sinv + n);
    float bb[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias) {
      const uint32_t b01 = *reinterpret_cast<const uint32_t*>(bias + n);
      const uint32_t b23 = *reinterpret_cast<const uint32_t*>(bias + n + 2);
      bb[0] = bf16_lo(b01); bb[1] = bf16_hi(b01); bb[2] = bf16_lo(b23); bb[3] = bf16_hi(b23);
    }
    const float y0 = fmaf(v[0] * sa, sb.x, bb[0]), y1 = fmaf(v[1] * sa, sb.y, bb[1]);
    const float y2 = fmaf(v[2] * sa, sb.z, bb[2]), y3 = fmaf(v[3] * sa, sb.w, bb[3]);
    *reinterpret_cast<uint2*>(C + (int64_t)m * ldc + n) = make_uint2(pack_bf16(y0, y1), pack_bf16(y2, y3));
  }
}

// Decode GEMM on fp16 operands (a16 already scaled and converted by the row pass,
// so neither operand needs VALU work): M up to a few hundred rows against a long
// weight stream. One block per R rows of b (R <= 64, chosen by the launcher so the
// blocks cover every CU once) and MT rows of a (grid.y = ceil(M / MT)). Both
// operands go global -> LDS by direct 16-byte buffer loads (buffer_load_dwordx4
// ... lds) into a ring of S k-tile stages, S - 1 tiles in flight per block and no
// VGPRs holding data in flight, so a CU keeps ~120 KB of loads outstanding; one
// barrier per k tile. LDS tile rows are 64 fp16 (128 bytes) with the 16-byte chunk
// index XOR-swizzled by (row / 2) % 8 (the direct loads apply the swizzle on the
// source side: lane j of a load lands at byte 16 j of its 1 KB block). MT <= 64:
// the four waves split each tile's four 16-wide k steps and their partial tiles
// are summed through LDS at the end; MT >= 128: each wave owns MT / 4 rows of a.
// Rows of b past R, rows of a past M and k past K load as zeros (past the end of
// the tile's buffer resource). The result is staged in LDS as bf16 rows and
// written in whole 16-byte lanes.
template <int MT, int S>
__global__ __launch_bounds__(256) void stream_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                     const float* __restrict__ a_sinv, const uint16_t* __restrict__ B,
                                                     int64_t ldb, const float* __restrict__ b_sinv,
                                                     const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
                                                     int64_t ldc, int M, int N, int K, int R) {
  constexpr int NP = 64;                      // LDS rows of b
  constexpr int STG = (MT + NP) * 128;        // one k tile of both operands
  constexpr int WK = MT <= 64 ? 4 : 1;        // waves splitting a tile's k steps
  constexpr int TM = MT * WK / 4;             // rows of a per wave
  constexpr int FM = TM / 32, FN = NP / 32;   // 32x32 MFMA blocks per wave
  constexpr int LW = (MT + NP) / 32;          // direct loads per wave per tile
  constexpr int LA = MT / 32;                 // the first LA of them are rows of a
  constexpr int OP = NP * 2 + 16;             // pitch of the bf16 output rows in LDS
  static_assert(S >= 3 && S <= 12 && MT % 32 == 0 && (WK == 1 || S >= 5), "stream shape");
  static_assert(FN * FM * 16 * 64 * 4 <= STG && MT * OP <= STG, "epilogue staging fits a stage");
  // one __shared__ object per stage: the compiler tracks direct-to-LDS loads per
  // object, so reading one stage never waits for the loads into the others
  __shared__ __align__(1024) uint8_t st0[STG], st1[STG], st2[STG];
  __shared__ __align__(1024) uint8_t st3[S > 3 ? STG : 16], st4[S > 4 ? STG : 16], st5[S > 5 ? STG : 16];
  __shared__ __align__(1024) uint8_t st6[S > 6 ? STG : 16], st7[S > 7 ? STG : 16], st8[S > 8 ? STG : 16];
  __shared__ __align__(1024) uint8_t st9[S > 9 ? STG : 16], st10[S > 10 ? STG : 16], st11[S > 11 ? STG : 16];
  uint8_t* const stages[12] = {st0, st1, st2, st3, st4, st5, st6, st7, st8, st9, st10, st11};

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * R, m0 = blockIdx.y * MT;
  const int nrows = min(R, N - n0), mrows = min(MT, M - m0);
  const BufRes ares = make_res(A + (int64_t)m0 * lda, (int64_t)mrows * lda * 2);
  const BufRes bres = make_res(B + (int64_t)n0 * ldb, (int64_t)nrows * ldb * 2);
  // load j of wave w fills 1 KB block w + 4 j of the stage: rows 8 (w + 4 j) + lane / 8
  // of the stacked [a rows | b rows] tile, physical chunk lane % 8, which holds
  // logical chunk `chunk` (the same for every load of this wave)
  const int chunk = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
  int voff[LW];
#pragma unroll
  for (int j = 0; j < LW; ++j) {
    const int row = 8 * (wave + 4 * j) + (lane >> 3);
    voff[j] = j < LA ? (row * (int)lda + chunk * 8) * 2 : ((row - MT) * (int)ldb + chunk * 8) * 2;
  }
  auto issue = [&](uint8_t* stage, int kt) {
    const uint32_t base = lds_addr(stage);
    const bool kok = kt * 64 + chunk * 8 < K;  // a k tail reads zeros (offset past any resource)
#pragma unroll
    for (int j = 0; j < LW; ++j)
      buf_load16_lds(j < LA ? ares : bres, base + (wave + 4 * j) * 1024, kok ? voff[j] : (int)0x80000000, kt * 128);
  };

  floatx16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int fr = lane & 31, fk = lane >> 5;
  const int wm = WK == 1 ? wave : 0;
  auto compute = [&](const uint8_t* stage) {
#pragma unroll
    for (int s = 0; s < 4 / WK; ++s) {
      const int c = 2 * (WK == 1 ? s : wave) + fk;
      half8 bf[FN], af[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) bf[i] = *reinterpret_cast<const half8*>(stage + swz<64>(MT + i * 32 + fr, c));
#pragma unroll
      for (int j = 0; j < FM; ++j) af[j] = *reinterpret_cast<const half8*>(stage + swz<64>(wm * TM + j * 32 + fr, c));
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], acc[i][j], 0, 0, 0);
    }
  };

  const int KT = (K + 63) / 64;
#pragma unroll
  for (int u = 0; u < S - 1; ++u)
    if (u < KT) issue(stages[u], u);
  for (int kt0 = 0; kt0 < KT; kt0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int kt = kt0 + u;
      if (kt < KT) {
        // this wave's loads of tile kt have landed once no more than the later
        // tiles' loads (up to S - 2 tiles, fewer at the end) are outstanding
        if (kt + S - 2 < KT) wait_vmem_n<LW * (S - 2)>();
        else wait_vmem_n<0>();
        // tile kt complete in LDS; every wave is past tile kt - 1 (a bare barrier:
        // __syncthreads' workgroup fence would wait for every load in flight)
        barrier_no_fence();
        if (kt + S - 1 < KT) issue(stages[(u + S - 1) % S], kt + S - 1);
        compute(stages[u]);
      }
    }
  }
  __syncthreads();  // the stages are reused below

  // ---- epilogue: (acc * sa[m]) * sb[n] + bias[n] -> bf16 rows in LDS -> C ----
  uint8_t* otile = WK > 1 ? st4 : st0;
  auto final_store = [&](int ml, int nl, const float (&v)[4]) {
    const int m = m0 + ml, n = n0 + nl;
    const float sa = m < M ? a_sinv[m] : 0.f;
    float4 sb = make_float4(0.f, 0.f, 0.f, 0.f);
    float bb[4] = {0.f, 0.f, 0.f, 0.f};
    if (nl < nrows) {
      sb = *reinterpret_cast<const float4*>(b_sinv + n);
      if (bias) {
        const uint32_t b01 = *reinterpret_cast<const uint32_t*>(bias + n);
        const uint32_t b23 = *reinterpret_cast<const uint32_t*>(bias + n + 2);
        bb[0] = bf16_lo(b01); bb[1] = bf16_hi(b01); bb[2] = bf16_lo(b23); bb[3] = bf16_hi(b23);
      }
    }
    const float y0 = fmaf(v[0] * sa, sb.x, bb[0]), y1 = fmaf(v[1] * sa, sb.y, bb[1]);
    const float y2 = fmaf(v[2] * sa, sb.z, bb[2]), y3 = fmaf(v[3] * sa, sb.w, bb[3]);
    *reinterpret_cast<uint2*>(otile + ml * OP + nl * 2) = make_uint2(pack_bf16(y0, y1), pack_bf16(y2, y3));
  };
  if constexpr (WK > 1) {
    // wave w's partial tile into stage w, then every thread sums four partials
    float* red = reinterpret_cast<float*>(wave == 0 ? st0 : wave == 1 ? st1 : wave == 2 ? st2 : st3);
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[((i * FM + j) * 16 + r) * 64 + lane] = acc[i][j][r];
    __syncthreads();
    const float* parts[4] = {reinterpret_cast<const float*>(st0), reinterpret_cast<const float*>(st1),
                             reinterpret_cast<const float*>(st2), reinterpret_cast<const float*>(st3)};
#pragma unroll
    for (int g = tid; g < FN * FM * 4 * 64; g += 256) {
      const int blk = g >> 8, rq = (g >> 6) & 3, ln = g & 63;
      const int i = blk / FM, j = blk % FM;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += parts[w][(blk * 16 + 4 * rq + e) * 64 + ln];
      final_store(j * 32 + (ln & 31), i * 32 + 8 * rq + 4 * (ln >> 5), v);
    }
  } else {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          final_store(wm * TM + j * 32 + fr, i * 32 + 8 * q + 4 * fk, v);
        }
  }
  __syncthreads();
  constexpr int OCR = NP / 8;  // 16-byte chunks per output row
  for (int g = tid; g < MT * OCR; g += 256) {
    const int ml = g / OCR, cc = g % OCR;
    if (ml < mrows && cc * 8 < nrows)
      stg16(C + (int64_t)(m0 + ml) * ldc + n0 + cc * 8, *reinterpret_cast<const uint4*>(otile + ml * OP + cc * 16));
  }
}

struct TileCfg {
  int bm, bn, bk;  // skinny configurations: bm = the largest M they take
  bool skinny;
  bool stream;  // fp16 a only (stream_kernel); bm = rows of a per block
};
// Tiled configurations (block tile, waves, k tile, register sets in flight, LDS stages):
// 0: 256x256, 8 waves of 64x128 (2 per SIMD), k 32, 3 sets, 3 stages, grouped MFMA schedule
// 1: 128x128, 4 waves of 64x64, k 64, 2 sets, 2 stages
// 2: 64x64, 4 waves of 32x32, k 64, 2 sets, 2 stages
// 3: 128x128, 4 waves of 64x64, k 64, 2 sets, 3 stages
// 4: 256x256, 8 waves of 64x128, k 32, 3 sets, 2 stages (no grouped schedule)
// Skinny configurations (M <= bm; 4 waves splitting K; block = 32 NB rows of b):
// 5: M <= 32, b registers-direct, 4 chunks in flight
// 6: M <= 32, b loaded coalesced and transposed through LDS, 4 chunks in flight
// 7: M <= 64, as 6 with 3 chunks in flight
// 8: M <= 64, 64 b rows per block, as 6 with 2 chunks in flight
// Two-stage k 64 loop with the last k step deferred past the barrier:
// 9: 256x256, 8 waves of 64x128, 1 set
// 10: 256x128, 8 waves of 64x64, 1 set
// 11: 256x64, 8 waves of 64x32, 3 sets (a k tile is only ~512 MFMA cycles here:
//     3 sets in flight 31.8 -> 30.2 us at M = 255, N = 10240, K = 2560; 4 or 6 slower)
// and 12: 128x64, 4 waves of 64x32, k 64, 3 sets, 3 stages
// Skinny, M <= 32: 13: 64 b rows per block, 8 waves splitting K, 3 chunks in flight
// Skinny, M <= 64: 14: 64 b rows per block, 8 waves splitting K, 1 chunk in flight
// Decode on fp16 a (stream_kernel, b rows spread over every CU, direct-to-LDS ring):
// 15: 32 rows of a, 12 stages; 16: 64 rows, 9 stages; 17: 128 rows, 6 stages;
// 18: 256 rows, 3 stages
// Two-stage k 64 loop as 9: 19: 192x256, 8 waves of 96x64 (a tile count that fills
// the CUs where 256-row tiles leave some idle, e.g. M = 6144: 32 rows of tiles)
constexpr TileCfg kCfgs[] = {{256, 256, 32}, {128, 128, 64}, {64, 64, 64},       {128, 128, 64},    {256, 256, 32},
                             {32, 32, 64, true}, {32, 32, 64, true}, {64, 32, 64, true}, {64, 64, 64, true},
                             {256, 256, 64}, {256, 128, 64}, {256, 64, 64}, {128, 64, 64}, {32, 64, 64, true},
                             {64, 64, 64, true}, {32, 64, 64, false, true}, {64, 64, 64, false, true},
                             {128, 64, 64, false, true}, {256, 64, 64, false, true},
                             {192, 256, 64}};
constexpr int kNumCfgs = 20;

// Compute units of the current device (cached per device).
int64_t num_cus() {
  static int64_t cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Configuration choice, fitted to measurements on MI355X (256 CUs). f16a: the caller
// can supply fp16 a (the decode configurations need it). Otherwise, for M <= 64
// with enough b rows for 160 blocks, the 64-row skinny block (8 waves splitting
// K, 3 chunks in flight: 17.6 -> 16.4 us at M = 16, K = 2560, N = 10240) up to M = 32 and
// the LDS-staged 64x64 tile above (every skinny block re-reads all of a, which
// costs more than the weights from M ~ 40 on). Otherwise the tile that maximises
// eff x (blocks / whole rounds of 256 blocks) x (M / M rounded up to the tile):
// larger tiles run faster per CU (eff), but a partial last round of blocks or a
// mostly empty row of tiles wastes CUs.
// Split K in two (tile configurations, workspace entry points): where a tile
// configuration leaves at least half the CUs without a tile, K >= 2048 and the
// fp32 partial sums take at most kSplitPartBytes, two blocks per tile each sum half
// of K into the workspace and a reduction applies the epilogue (256x4096x4096:
// 128 tiles of 128x64 -> 256 blocks). The output differs from the unsplit one only
// by the order of the fp32 additions (exact for integer-valued products).
constexpr size_t kSplitPartBytes = (size_t)8 << 20;
int pick_split(int cfg, int64_t M, int64_t N, int64_t K) {
  if (cfg < 0 || cfg >= kNumCfgs || kCfgs[cfg].skinny || kCfgs[cfg].stream || K < 2048) return 1;
  const int64_t tiles = cdiv(M, kCfgs[cfg].bm) * cdiv(N, kCfgs[cfg].bn);
  if (2 * tiles > num_cus() || (size_t)2 * (size_t)M * (size_t)N * 4 > kSplitPartBytes) return 1;
  return 2;
}

// K > 0: the caller can split K (pick_split), which the score accounts for.
int pick_cfg(int64_t M, int64_t N, bool f16a, int64_t K = 0) {
  // decode on fp16 a (a16 given, or tbf16_linear's workspace copy): the direct-to-LDS
  // ring for M <= 128 once N fills every CU with at least 32 b rows (M = 16 / 64 /
  // 128 at K = 2560, N = 10240: 13.3 / 18.2 / 23.0 us against 13.6 / 24.1 / 26.9 for
  // the kernels below; at M = 255 the two tie, and the 256-row tiles skip the copy)
  if (f16a && M <= 128 && N >= 32 * num_cus()) return M <= 32 ? 15 : M <= 64 ? 16 : 17;
  if (M <= 64) {
    if (cdiv(N, 64) >= 160) return M <= 32 ? 13 : 2;
    return M <= 32 ? 6 : 7;
  }
  const int64_t kCUs = num_cus();
  // eff of the 192x256 tile: 179.1 us for 6144x2048x8192 against 170.4 us for the
  // 256x256 tile on 8192x2048x6144 (both one tile per CU, the same flops per CU)
  constexpr int cand[] = {9, 19, 10, 11, 12, 2};
  constexpr float eff[] = {1.0f, 0.95f, 0.85f, 0.7f, 0.6f, 0.45f};
  constexpr int ncand = sizeof(cand) / sizeof(cand[0]);
  int best = 2;
  float best_score = -1.f;
  for (int i = 0; i < ncand; ++i) {
    const TileCfg& t = kCfgs[cand[i]];
    const int s = K > 0 ? pick_split(cand[i], M, N, K) : 1;
    const int64_t mt = cdiv(M, t.bm), tiles = mt * cdiv(N, t.bn) * s;
    const float util = (float)tiles / (float)(cdiv(tiles, kCUs) * kCUs);
    const float mutil = (float)M / (float)(mt * t.bm);
    // the partial sums' round trip and the reduction launch: 0.9 (17.3 + ~3 us
    // against 25.2 us unsplit for 256x4096x4096)
    const float score = eff[i] * util * mutil * (s > 1 ? 0.9f : 1.0f);
    if (score > best_score) {
      best_score = score;
      best = cand[i];
    }
  }
  return best;
}

template <int BM, int BN, int WM, int WN, int BK, int PF, int NS, bool A_BF16>
void launch_cfg(bool even, unsigned blocks, const uint16_t* a, int64_t lda, const int32_t* a_exp, const float* a_sinv,
                const uint16_t* b, int64_t ldb, const float* b_sinv, const uint16_t* bi, uint16_t* c, int64_t ldc,
                int M, int N, int K, float* part, int splits, hipStream_t st) {
  const int kt_per = (int)cdiv(cdiv(K, BK), splits);
  const dim3 grid(blocks, part ? (unsigned)splits : 1u);
  if (even)
    gemm_kernel<BM, BN, WM, WN, BK, PF, NS, A_BF16, true><<<grid, WM * WN * 64, 0, st>>>(a, lda, a_exp, a_sinv, b, ldb, b_sinv,
                                                                             bi, c, ldc, M, N, K, part, kt_per);
  else
    gemm_kernel<BM, BN, WM, WN, BK, PF, NS, A_BF16, false><<<grid, WM * WN * 64, 0, st>>>(a, lda, a_exp, a_sinv, b, ldb, b_sinv,
                                                                              bi, c, ldc, M, N, K, part, kt_per);
}

// part / splits: split K over `splits` blocks per tile (tile configurations only),
// the fp32 partial sums in part (splits x M x N), then splitk_reduce_kernel.
template <bool A_BF16>
int launch_gemm(int cfg, const void* A, int64_t lda, const int32_t* a_exp, const float* a_sinv, const void* B,
                int64_t ldb, const float* b_sinv, const void* bias, void* C, int64_t ldc, int64_t M, int64_t N,
                int64_t K, hipStream_t st, float* part = nullptr, int splits = 1) {
  const int bm = kCfgs[cfg].bm, bn = kCfgs[cfg].bn;
  TB_CHECK(splits == 1 || (part != nullptr && splits > 1 && !kCfgs[cfg].skinny && !kCfgs[cfg].stream &&
                           (int64_t)splits * kCfgs[cfg].bk <= K),
           "gemm: split K needs a tile configuration, a partial-sum buffer and K >= splits k tiles");
  if (splits == 1) part = nullptr;
  TB_CHECK(!kCfgs[cfg].skinny || M <= bm, "gemm: configuration %d takes M <= %d", cfg, bm);
  TB_CHECK(!kCfgs[cfg].stream || !A_BF16, "gemm: configuration %d needs fp16 a (tbf16_gemm_f16 or tbf16_linear)", cfg);
  // skinny and stream blocks take `rows` weight rows each: as many as fit (bn)
  // when that already fills whole rounds of blocks over the CUs, else fewer, so
  // that the weight stream is spread over every CU in as few rounds as possible
  int rows = bn;
  if (kCfgs[cfg].skinny || kCfgs[cfg].stream) {
    const int64_t ncu = num_cus();
    const int64_t rounds = cdiv(cdiv(N, bn), ncu);
    rows = (int)std::min<int64_t>(bn, std::max<int64_t>(8, cdiv(cdiv(N, rounds * ncu), 8) * 8));
  }
  const int64_t blocks = kCfgs[cfg].skinny || kCfgs[cfg].stream ? cdiv(N, rows) : cdiv(M, bm) * cdiv(N, bn);
  TB_CHECK(blocks < (int64_t)1 << 31 && cdiv(M, bm) < 65536, "gemm: grid too large");
  const bool even = K % kCfgs[cfg].bk == 0;  // no k-tail selects on loaded values
  const auto a = (const uint16_t*)A;
  const auto b = (const uint16_t*)B;
  const auto bi = (const uint16_t*)bias;
  const auto c = (uint16_t*)C;
  const unsigned g = (unsigned)blocks;
  switch (cfg) {
#define CFG(BM_, BN_, WM_, WN_, BK_, PF_, NS_)                                                                       \
  launch_cfg<BM_, BN_, WM_, WN_, BK_, PF_, NS_, A_BF16>(even, g, a, lda, a_exp, a_sinv, b, ldb, b_sinv, bi, c, ldc, M, N, K, \
                                                        part, splits, st)
    case 0: CFG(256, 256, 4, 2, 32, 3, 4); break;
    case 1: CFG(128, 128, 2, 2, 64, 2, 2); break;
    case 2: CFG(64, 64, 2, 2, 64, 2, 2); break;
    case 3: CFG(128, 128, 2, 2, 64, 2, 3); break;
    case 4: CFG(256, 256, 4, 2, 32, 3, 2); break;
    case 9: CFG(256, 256, 4, 2, 64, 1, 5); break;
    case 10: CFG(256, 128, 4, 2, 64, 1, 5); break;
    case 11: CFG(256, 64, 4, 2, 64, 3, 5); break;
    case 12: CFG(128, 64, 2, 2, 64, 3, 3); break;
    case 19: CFG(192, 256, 2, 4, 64, 1, 5); break;
#define SKINNY(NB_, MB_, NW_, PF_, TR_)                                                                         \
  skinny_kernel<NB_, MB_, NW_, PF_, TR_, A_BF16><<<g, NW_ * 64, 0, st>>>(a, lda, a_exp, a_sinv, b, ldb, b_sinv, bi, c, \
                                                                        ldc, M, N, K, rows)
    case 5: SKINNY(1, 1, 4, 4, false); break;
    case 6: SKINNY(1, 1, 4, 4, true); break;
    case 7: SKINNY(1, 2, 4, 3, true); break;
    case 13: SKINNY(2, 1, 8, 3, true); break;
    case 14: SKINNY(2, 2, 8, 1, true); break;
#define STREAM(MT_, S_)                                                                                  \
  if constexpr (!A_BF16)                                                                                 \
    stream_kernel<MT_, S_><<<dim3(g, (unsigned)cdiv(M, MT_)), 256, 0, st>>>(a, lda, a_sinv, b, ldb, b_sinv, bi, c, \
                                                                          ldc, M, N, K, rows)
    case 15: STREAM(32, 12); break;
    case 16: STREAM(64, 9); break;
    case 17: STREAM(128, 6); break;
    case 18: STREAM(256, 3); break;
    default: SKINNY(2, 2, 4, 2, true); break;
#undef STREAM
#undef SKINNY
#undef CFG
  }
  TB_LAUNCH_CHECK("gemm");
  if (part) {
    const int64_t groups = M * (N / 8);
    splitk_reduce_kernel<A_BF16><<<(unsigned)cdiv(groups, 256), 256, 0, st>>>(part, splits, a_exp, a_sinv, b_sinv, bi, c,
                                                                             ldc, (int)M, (int)N);
    TB_LAUNCH_CHECK("gemm split-K reduction");
  }
  return 0;
}

int check_gemm(const char* fn, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B,
               int64_t ldb, const float* sb, const void* bias, const void* C, int64_t ldc) {
  TB_CHECK(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", fn);
  TB_CHECK(M < (int64_t)1 << 31 && N < (int64_t)1 << 31 && K < (int64_t)1 << 31, "%s: shape too large", fn);
  TB_CHECK(K % 8 == 0 && N % 8 == 0, "%s: N and K must be multiples of 8", fn);
  TB_CHECK(lda % 8 == 0 && lda >= K && ldb % 8 == 0 && ldb >= K && ldc % 8 == 0 && ldc >= N,
           "%s: row strides must be multiples of 8", fn);
  TB_CHECK(aligned16(A) && aligned16(B) && aligned16(C) && aligned16(sb), "%s: operands must be 16-byte aligned", fn);
  TB_CHECK(bias == nullptr || aligned4(bias), "%s: bias must be 4-byte aligned", fn);
  // tile row offsets are 32-bit byte offsets from the tile's first row
  TB_CHECK(lda < (int64_t)1 << 22 && ldb < (int64_t)1 << 22, "%s: row stride too large", fn);
  return 0;
}

}  // namespace

namespace tbf16 {
int launch_row_exps(const void* x, int64_t M, int64_t K, int64_t ldx, int t, int l1, int32_t* exps, float* s_inv,
                    hipStream_t st);
int launch_quantize_rows(const void* x, int64_t R, int64_t K, int64_t ldx, int t, int l1, void* y16, int64_t ldy,
                         float* s_inv, int32_t* exps, hipStream_t st);
}  // namespace tbf16

namespace {

// Whether tbf16_linear quantises x once (row exponents, inverse scales and the
// fp16 rows into its workspace) and runs the GEMM on fp16 operands, instead of
// converting x inside the GEMM. The decode kernel takes fp16 a only. Tiles of at
// most 128 columns convert each x tile once per column block (64 times at N =
// 4096 with 64-column tiles), which the one pass saves: bit-identical output,
// 256x4096x4096 34.6 -> 27.7 us, 1024x4096x4096 56.9 -> 50.3, 2048x4096x4096 84.4
// -> 77.1 (128-column tiles). 256-column tiles convert x 16 times at N = 4096
// and gain nothing there (4096^3: the extra pass costs more than it saves), and
// at K < 1024 the pass costs about what it saves (200x2560x768: 10.0 vs 10.6 us).
bool quantize_once(int cfg, int64_t K) {
  if (cfg < 0 || cfg >= kNumCfgs) return false;
  const TileCfg& c = kCfgs[cfg];
  return c.stream || (!c.skinny && c.bn <= 128 && K >= 1024);
}

// Workspace of tbf16_linear: the row exponents (int32 (M,)); where x is quantised
// once (`quantize_once`, unless `fused` asks for the conversion inside the GEMM,
// which the decode kernel cannot do), the row inverse scales (fp32 (M,)) and the
// scaled fp16 copy of x (M, K); where K is split (`pick_split`), the fp32 partial
// sums (splits x M x N). Each part 256-byte aligned.
struct LinearWs {
  size_t exps, sinv, x16, part, bytes;
  int splits;
  bool q16;
};
LinearWs linear_ws(int64_t M, int64_t K, int64_t N, int cfg, bool fused = false) {
  LinearWs w{0, 0, 0, 0, align_up((size_t)M * 4, 256), 1, false};
  w.q16 = quantize_once(cfg, K) && !(fused && !kCfgs[cfg].stream);
  if (w.q16) {
    w.sinv = w.bytes;
    w.x16 = w.sinv + align_up((size_t)M * 4, 256);
    w.bytes = align_up(w.x16 + (size_t)M * (size_t)K * 2, 256);
  }
  w.splits = pick_split(cfg, M, N, K);
  if (w.splits > 1) {
    w.part = w.bytes;
    w.bytes = w.part + (size_t)w.splits * (size_t)M * (size_t)N * 4;
  }
  return w;
}

// fused: convert x inside the GEMM even where `quantize_once` holds (same output;
// for a workspace too small for the fp16 copy of x). The decode kernel cannot.
int linear_into(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w16, int64_t N, int64_t ldw,
                const float* ws, const void* bias, void* y, int64_t ldy, int t, int l1, int cfg, uint8_t* wsp,
                bool fused, hipStream_t st) {
  const LinearWs w = linear_ws(M, K, N, cfg, fused);
  int32_t* exps = reinterpret_cast<int32_t*>(wsp + w.exps);
  float* part = w.splits > 1 ? reinterpret_cast<float*>(wsp + w.part) : nullptr;
  if (!w.q16) {
    if (int rc = launch_row_exps(x, M, K, ldx, t, l1, exps, nullptr, st)) return rc;
    return launch_gemm<true>(cfg, x, ldx, exps, nullptr, w16, ldw, ws, bias, y, ldy, M, N, K, st, part, w.splits);
  }
  // x quantised once (exponents, inverse scales, fp16 rows), then the GEMM on fp16
  // operands: the same fp16 values the fused kernels convert in registers
  float* sinv = reinterpret_cast<float*>(wsp + w.sinv);
  void* x16 = wsp + w.x16;
  if (int rc = launch_quantize_rows(x, M, K, ldx, t, l1, x16, K, sinv, exps, st)) return rc;
  return launch_gemm<false>(cfg, x16, K, nullptr, sinv, w16, ldw, ws, bias, y, ldy, M, N, K, st, part, w.splits);
}
}  // namespace

extern "C" size_t tbf16_linear_ws_bytes(int64_t M, int64_t K, int64_t N, int cfg) {
  if (M <= 0 || K < 0 || N <= 0 || cfg >= kNumCfgs) return M > 0 ? (size_t)M * 4 : 0;
  return linear_ws(M, K, N, cfg < 0 ? pick_cfg(M, N, true, K) : cfg).bytes;
}

extern "C" int tbf16_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w16, int64_t N,
                            int64_t ldw, const float* ws, const void* bias, void* y, int64_t ldy, int t, int l1,
                            int cfg, void* workspace, void* stream) {
  if (int rc = check_gemm("linear", M, N, K, x, ldx, w16, ldw, ws, bias, y, ldy)) return rc;
  TB_CHECK(workspace != nullptr || M == 0, "linear: workspace missing");
  TB_CHECK(aligned16(workspace), "linear: workspace must be 16-byte aligned");
  TB_CHECK(cfg < kNumCfgs, "bad cfg");
  if (M == 0 || N == 0) return 0;
  return linear_into(x, M, K, ldx, w16, N, ldw, ws, bias, y, ldy, t, l1, cfg < 0 ? pick_cfg(M, N, true, K) : cfg,
                     static_cast<uint8_t*>(workspace), false, as_stream(stream));
}

// ---- tbf16_linear_noalloc: the workspace in a static device array ---------------
// Each GPU the library runs on holds one copy of `scratch` (TBF16_NOALLOC_SCRATCH_BYTES)
// until the process ends. Host code never passes the array's name to a kernel (on
// the host it is only a stand-in symbol): the device address of this GPU's copy
// comes from hipGetSymbolAddress, taken once per device with that device current,
// and is what the kernels get. Every call on one GPU shares the array, and the row
// pass (and, with split K, the GEMM's partial sums) overwrites exactly the parts a
// call uses before they are read, so nothing needs clearing; calls that overlap on
// one GPU (several streams or threads) race.
static __device__ __align__(256) uint8_t scratch[TBF16_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices] = {};

int scratch_ptr(uint8_t** out) {
  int dev = -1;
  TB_CHECK(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices, "linear_noalloc: no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    TB_CHECK(e == hipSuccess && p != nullptr, "linear_noalloc: hipGetSymbolAddress failed (%s)", hipGetErrorString(e));
    g_scratch[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch[dev];
  return 0;
}
}  // namespace

extern "C" int tbf16_linear_noalloc(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w16, int64_t N,
                                    int64_t ldw, const float* ws, const void* bias, void* y, int64_t ldy, int t,
                                    int l1, int cfg, void* stream) {
  TB_CHECK(M <= TBF16_NOALLOC_MAX_ROWS, "linear_noalloc: M = %lld rows exceeds the scratch limit of %d rows",
           (long long)M, TBF16_NOALLOC_MAX_ROWS);
  if (int rc = check_gemm("linear_noalloc", M, N, K, x, ldx, w16, ldw, ws, bias, y, ldy)) return rc;
  TB_CHECK(cfg < kNumCfgs, "bad cfg");
  if (M == 0 || N == 0) return 0;
  // the scratch address is this device's: the stream must run on it
  hipStream_t st = as_stream(stream);
  if (st != nullptr) {
    int cur = -1;
    hipDevice_t sd = -1;
    TB_CHECK(hipGetDevice(&cur) == hipSuccess && hipStreamGetDevice(st, &sd) == hipSuccess,
             "linear_noalloc: cannot query the stream's device");
    TB_CHECK(sd == cur, "linear_noalloc: the stream belongs to device %d, the current device is %d", (int)sd, cur);
  }
  const int c = cfg < 0 ? pick_cfg(M, N, true, K) : cfg;
  // where the fp16 copy of x does not fit, a tile configuration converts x inside
  // the GEMM instead (the same output); the decode kernel needs the copy
  const bool fused = !kCfgs[c].stream && linear_ws(M, K, N, c).bytes > TBF16_NOALLOC_SCRATCH_BYTES;
  const size_t need = linear_ws(M, K, N, c, fused).bytes;
  TB_CHECK(need <= TBF16_NOALLOC_SCRATCH_BYTES,
           "linear_noalloc: %lld x %lld needs %zu workspace bytes, beyond the scratch limit of %d bytes", (long long)M,
           (long long)K, need, TBF16_NOALLOC_SCRATCH_BYTES);
  uint8_t* wsp = nullptr;
  if (int rc = scratch_ptr(&wsp)) return rc;
  return linear_into(x, M, K, ldx, w16, N, ldw, ws, bias, y, ldy, t, l1, c, wsp, fused, st);
}

extern "C" int tbf16_linear_exps(const void* x, int64_t M, int64_t K, int64_t ldx, const int32_t* exps,
                                 const void* w16, int64_t N, int64_t ldw, const float* ws, const void* bias, void* y,
                                 int64_t ldy, int cfg, void* stream) {
  if (int rc = check_gemm("linear_exps", M, N, K, x, ldx, w16, ldw, ws, bias, y, ldy)) return rc;
  TB_CHECK(exps != nullptr || M == 0, "linear_exps: exps missing");
  TB_CHECK(cfg < kNumCfgs, "bad cfg");
  if (M == 0 || N == 0) return 0;
  return launch_gemm<true>(cfg < 0 ? pick_cfg(M, N, false) : cfg, x, ldx, exps, nullptr, w16, ldw, ws, bias, y, ldy, M, N, K,
                           as_stream(stream));
}

extern "C" int tbf16_gemm_f16(const void* a16, int64_t M, int64_t K, int64_t lda, const float* sa, const void* b16,
                              int64_t N, int64_t ldb, const float* sb, const void* bias, void* y, int64_t ldy, int cfg,
                              void* stream) {
  if (int rc = check_gemm("gemm_f16", M, N, K, a16, lda, b16, ldb, sb, bias, y, ldy)) return rc;
  TB_CHECK(sa != nullptr || M == 0, "gemm_f16: sa missing");
  TB_CHECK(cfg < kNumCfgs, "bad cfg");
  if (M == 0 || N == 0) return 0;
  return launch_gemm<false>(cfg < 0 ? pick_cfg(M, N, true) : cfg, a16, lda, nullptr, sa, b16, ldb, sb, bias, y, ldy, M, N,
                            K, as_stream(stream));
}
