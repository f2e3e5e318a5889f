// Scaled GEMM on CDNA4 fp16 MFMA: y = bf16(acc * sa[m] * sb[n] + bias[n]) with
// acc[m, n] = sum_k a16[m, k] * b16[n, k] in fp32.
//
// a is either already fp16 (a16 with fp32 inverse row scales sa) or bf16 that is
// converted to fp16 with an exact per-row power of two 2^p[m] on its way from
// registers into LDS, sa = 2^-p[m] (the fused path, tbf16/csrc/gemm_sm75.cu:78-226).
// b is fp16 (prepare_weight's w16) with fp32 inverse row scales sb.
//
// Tiling (gfx950, 64-wide waves, 160 KB LDS):
//  - block tile BM (rows of a) x BN (rows of b), k tile 64; WM x WN waves, each
//    owning a (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks
//    (v_mfma_f32_32x32x16_f16: 16 fp32 accumulators per lane per block).
//  - operands staged global -> VGPR -> LDS with 16-byte loads, two LDS stages and
//    the next k tile's loads in flight during the current tile's MFMAs; one
//    barrier per k tile. LDS rows are 128 bytes (64 fp16) with the 16-byte chunk
//    index XOR-swizzled by (row / 2) % 8, so the 32-row fragment reads
//    (ds_read_b128) and the 8-lanes-per-row stores are bank-conflict free.
//  - the MFMA's first operand is the b fragment, the second the a fragment, so a
//    lane's 16 accumulators are four runs of 4 consecutive n for one m: the
//    epilogue writes 8-byte bf16 runs straight from registers (one rounding).
//  - block ids are remapped so that each XCD (8 per chip, round-robin dispatch)
//    gets a contiguous range of tiles, grouped 8 a-tiles deep for L2 reuse.
#include <algorithm>

#include "abi_util.h"
#include "common.h"

using namespace tbf16;

namespace {

constexpr int BK = 64;

__device__ __forceinline__ int swz(int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); }

template <int BM, int BN, int WM, int WN, bool A_BF16>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                           const int32_t* __restrict__ a_exp,
                                                           const float* __restrict__ a_sinv,
                                                           const uint16_t* __restrict__ B, int64_t ldb,
                                                           const float* __restrict__ b_sinv,
                                                           const uint16_t* __restrict__ bias,
                                                           uint16_t* __restrict__ C, int64_t ldc, int M, int N, int K) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int RP = NT / 8;  // rows covered by one pass of 16-byte loads (8 lanes per 128-byte row)
  constexpr int AL = BM / RP, BL = BN / RP;
  static_assert(FM >= 1 && FN >= 1 && AL * RP == BM && BL * RP == BN, "bad tile");
  constexpr int STAGE = (BM + BN) * 128;
  __shared__ __align__(16) uint8_t smem[2 * STAGE];

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

  // ---- global -> register staging ----
  const int lrow = tid >> 3, lch = tid & 7;
  const uint16_t* ga[AL];
  const uint16_t* gb[BL];
  bool aok[AL], bok[BL];
  float as[AL];
#pragma unroll
  for (int i = 0; i < AL; ++i) {
    const int r = m0 + lrow + i * RP;
    aok[i] = r < M;
    ga[i] = A + (int64_t)(aok[i] ? r : 0) * lda + lch * 8;
    if constexpr (A_BF16) as[i] = aok[i] ? pow2f(a_exp[r]) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < BL; ++i) {
    const int r = n0 + lrow + i * RP;
    bok[i] = r < N;
    gb[i] = B + (int64_t)(bok[i] ? r : 0) * ldb + lch * 8;
  }
  uint4 ra[AL], rb[BL];
  auto gload = [&](int kt) {
    const bool kok = kt * BK + lch * 8 < K;
#pragma unroll
    for (int i = 0; i < AL; ++i) ra[i] = (kok && aok[i]) ? ldg16(ga[i] + kt * BK) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < BL; ++i) rb[i] = (kok && bok[i]) ? ldg16(gb[i] + kt * BK) : make_uint4(0, 0, 0, 0);
  };
  auto lstore = [&](int stg) {
    uint8_t* sA = smem + stg * STAGE;
    uint8_t* sB = sA + BM * 128;
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      uint4 v = ra[i];
      if constexpr (A_BF16) v = cvt_bf16x8_f16x8(v, as[i]);
      *reinterpret_cast<uint4*>(sA + swz(lrow + i * RP, lch)) = v;
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) *reinterpret_cast<uint4*>(sB + swz(lrow + i * RP, lch)) = rb[i];
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
    const uint8_t* sB = sA + BM * 128;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int c = 2 * s + fk;
      half8 bf[FN], af[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) bf[i] = *reinterpret_cast<const half8*>(sB + swz(wn * TN + i * 32 + fr, c));
#pragma unroll
      for (int j = 0; j < FM; ++j) af[j] = *reinterpret_cast<const half8*>(sA + swz(wm * TM + j * 32 + fr, c));
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], acc[i][j], 0, 0, 0);
    }
  };

  const int KT = (K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) gload(kt + 1);
    compute(kt & 1);
    if (kt + 1 < KT) lstore((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: (acc * sa[m]) * sb[n] + bias[n] -> bf16, 8-byte runs ----
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + wm * TM + j * 32 + fr;
    if (m >= M) continue;
    float sa;
    if constexpr (A_BF16) sa = ldexp1(-a_exp[m]);
    else sa = a_sinv[m];
    uint16_t* crow = C + (int64_t)m * ldc;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * TN + i * 32 + 8 * q + 4 * fk;
        if (n >= N) continue;
        const float4 sb = *reinterpret_cast<const float4*>(b_sinv + n);
        float bb[4] = {0.f, 0.f, 0.f, 0.f};
        if (bias) {
          const uint32_t b01 = *reinterpret_cast<const uint32_t*>(bias + n);
          const uint32_t b23 = *reinterpret_cast<const uint32_t*>(bias + n + 2);
          bb[0] = bf16_lo(b01); bb[1] = bf16_hi(b01); bb[2] = bf16_lo(b23); bb[3] = bf16_hi(b23);
        }
        const float y0 = fmaf(acc[i][j][4 * q + 0] * sa, sb.x, bb[0]);
        const float y1 = fmaf(acc[i][j][4 * q + 1] * sa, sb.y, bb[1]);
        const float y2 = fmaf(acc[i][j][4 * q + 2] * sa, sb.z, bb[2]);
        const float y3 = fmaf(acc[i][j][4 * q + 3] * sa, sb.w, bb[3]);
        *reinterpret_cast<uint2*>(crow + n) = make_uint2(pack_bf16(y0, y1), pack_bf16(y2, y3));
      }
    }
  }
}

struct TileCfg {
  int bm, bn;
};
constexpr TileCfg kCfgs[] = {{256, 256}, {128, 128}, {64, 64}, {64, 32}};
constexpr int kNumCfgs = 4;

int pick_cfg(int64_t M, int64_t N) {
  auto tiles = [&](int c) { return cdiv(M, kCfgs[c].bm) * cdiv(N, kCfgs[c].bn); };
  if (tiles(0) >= 192) return 0;
  if (tiles(1) >= 160) return 1;
  if (M <= 64) return 3;
  return 2;
}

template <bool A_BF16>
int launch_gemm(int cfg, const void* A, int64_t lda, const int32_t* a_exp, const float* a_sinv, const void* B,
                int64_t ldb, const float* b_sinv, const void* bias, void* C, int64_t ldc, int64_t M, int64_t N,
                int64_t K, hipStream_t st) {
  const int64_t blocks = cdiv(M, kCfgs[cfg].bm) * cdiv(N, kCfgs[cfg].bn);
  TB_CHECK(blocks < (int64_t)1 << 31, "gemm: grid too large");
  const auto a = (const uint16_t*)A;
  const auto b = (const uint16_t*)B;
  const auto bi = (const uint16_t*)bias;
  const auto c = (uint16_t*)C;
  switch (cfg) {
    case 0:
      gemm_kernel<256, 256, 4, 2, A_BF16><<<(unsigned)blocks, 512, 0, st>>>(a, lda, a_exp, a_sinv, b, ldb, b_sinv, bi, c,
                                                                            ldc, (int)M, (int)N, (int)K);
      break;
    case 1:
      gemm_kernel<128, 128, 2, 2, A_BF16><<<(unsigned)blocks, 256, 0, st>>>(a, lda, a_exp, a_sinv, b, ldb, b_sinv, bi, c,
                                                                            ldc, (int)M, (int)N, (int)K);
      break;
    case 2:
      gemm_kernel<64, 64, 2, 2, A_BF16><<<(unsigned)blocks, 256, 0, st>>>(a, lda, a_exp, a_sinv, b, ldb, b_sinv, bi, c,
                                                                          ldc, (int)M, (int)N, (int)K);
      break;
    default:
      gemm_kernel<64, 32, 1, 1, A_BF16><<<(unsigned)blocks, 64, 0, st>>>(a, lda, a_exp, a_sinv, b, ldb, b_sinv, bi, c,
                                                                         ldc, (int)M, (int)N, (int)K);
      break;
  }
  TB_LAUNCH_CHECK("gemm");
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
  return 0;
}

}  // namespace

namespace tbf16 {
int launch_row_exps(const void* x, int64_t M, int64_t K, int64_t ldx, int t, int l1, int32_t* exps, float* s_inv,
                    hipStream_t st);
}

extern "C" int tbf16_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w16, int64_t N,
                            int64_t ldw, const float* ws, const void* bias, void* y, int64_t ldy, int t, int l1,
                            int cfg, int32_t* exps_ws, void* stream) {
  if (int rc = check_gemm("linear", M, N, K, x, ldx, w16, ldw, ws, bias, y, ldy)) return rc;
  TB_CHECK(exps_ws != nullptr || M == 0, "linear: exps workspace missing");
  TB_CHECK(cfg < kNumCfgs, "bad cfg");
  if (M == 0 || N == 0) return 0;
  hipStream_t st = as_stream(stream);
  if (int rc = launch_row_exps(x, M, K, ldx, t, l1, exps_ws, nullptr, st)) return rc;
  return launch_gemm<true>(cfg < 0 ? pick_cfg(M, N) : cfg, x, ldx, exps_ws, nullptr, w16, ldw, ws, bias, y, ldy, M, N,
                           K, st);
}

extern "C" int tbf16_linear_exps(const void* x, int64_t M, int64_t K, int64_t ldx, const int32_t* exps,
                                 const void* w16, int64_t N, int64_t ldw, const float* ws, const void* bias, void* y,
                                 int64_t ldy, int cfg, void* stream) {
  if (int rc = check_gemm("linear_exps", M, N, K, x, ldx, w16, ldw, ws, bias, y, ldy)) return rc;
  TB_CHECK(exps != nullptr || M == 0, "linear_exps: exps missing");
  TB_CHECK(cfg < kNumCfgs, "bad cfg");
  if (M == 0 || N == 0) return 0;
  return launch_gemm<true>(cfg < 0 ? pick_cfg(M, N) : cfg, x, ldx, exps, nullptr, w16, ldw, ws, bias, y, ldy, M, N, K,
                           as_stream(stream));
}

extern "C" int tbf16_gemm_f16(const void* a16, int64_t M, int64_t K, int64_t lda, const float* sa, const void* b16,
                              int64_t N, int64_t ldb, const float* sb, const void* bias, void* y, int64_t ldy, int cfg,
                              void* stream) {
  if (int rc = check_gemm("gemm_f16", M, N, K, a16, lda, b16, ldb, sb, bias, y, ldy)) return rc;
  TB_CHECK(sa != nullptr || M == 0, "gemm_f16: sa missing");
  TB_CHECK(cfg < kNumCfgs, "bad cfg");
  if (M == 0 || N == 0) return 0;
  return launch_gemm<false>(cfg < 0 ? pick_cfg(M, N) : cfg, a16, lda, nullptr, sa, b16, ldb, sb, bias, y, ldy, M, N,
                            K, as_stream(stream));
}
