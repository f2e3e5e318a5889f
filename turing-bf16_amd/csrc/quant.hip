// Memory-bound kernels of the hot path: row / column power-of-two scaling and
// quantisation to fp16, per-head amax and scale-cast, and the M = 1 GEMV.
//
// All of them stream HBM once (twice for the two-pass row quantiser, whose
// second read hits L2). Loads and stores are 16 bytes per lane; one wave
// (64 lanes) owns a row where rows are long, so reductions are in-wave.
#include <algorithm>

#include "abi_util.h"
#include "common.h"

using namespace tbf16;

namespace {

constexpr int kRowWaves = 4;  // rows per 256-thread block
// quantize_rows reads rows of up to kRegChunks x 512 elements into registers, every
// load issued before the reduction, and converts them from there.
constexpr int kRegChunks = 16;

// amax (or L1 norm) of a row held in v[] (16-byte chunks lane + 64 c, zeros past
// K8): the same element order and arithmetic as row_amax_wave, so the same bits.
__device__ __forceinline__ float row_amax_regs(const uint4 (&v)[kRegChunks], int K8, int lane, bool l1) {
  if (l1) {
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < kRegChunks; ++c)
      if (lane + c * kWave < K8) acc += l1_chunk(v[c]);
    return (float)wave_sum_d(acc);
  }
  float m = 0.f;  // zero chunks past the row end leave the maximum alone
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c)
    m = fmaxf(m, fmaxf(fmaxf(fmaxf(fabsf(bf16_lo(v[c].x)), fabsf(bf16_hi(v[c].x))),
                             fmaxf(fabsf(bf16_lo(v[c].y)), fabsf(bf16_hi(v[c].y)))),
                       fmaxf(fmaxf(fabsf(bf16_lo(v[c].z)), fabsf(bf16_hi(v[c].z))),
                             fmaxf(fabsf(bf16_lo(v[c].w)), fabsf(bf16_hi(v[c].w))))));
  return wave_max(m);
}
__device__ __forceinline__ void load_row_regs(const uint4* src, int K8, int lane, uint4 (&v)[kRegChunks]) {
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) v[c] = lane + c * kWave < K8 ? src[lane + c * kWave] : make_uint4(0, 0, 0, 0);
}

// Row exponents: one wave per row (gemm_sm75.cu:27-47 does one warp per row).
__global__ __launch_bounds__(256) void row_exps_kernel(const uint16_t* __restrict__ x, int64_t M, int K, int64_t ldx,
                                                       int t, int l1, int32_t* __restrict__ exps,
                                                       float* __restrict__ s_inv) {
  const int64_t row = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  // (the loop form: holding the row in registers as quantize_rows does ran slower
  // here, 4.8 -> 6.7 us at 4096 x 4096, with nothing to reuse the registers for)
  const float amax = row_amax_wave(x + row * ldx, K, lane, l1 != 0);
  if (lane == 0) {
    const int p = pow2_exp(amax, t);
    if (exps) exps[row] = p;
    if (s_inv) s_inv[row] = ldexp1(-p);
  }
}

// quantize_rows: amax pass, then y = fp16(x * 2^p) (small_kernels.cu:35-74).
// Rows of up to kRegChunks x 512 elements are read once, into registers.
__global__ __launch_bounds__(256) void quantize_rows_kernel(const uint16_t* __restrict__ x, int64_t R, int K,
                                                            int64_t ldx, int t, int l1, uint16_t* __restrict__ y,
                                                            int64_t ldy, float* __restrict__ s_inv,
                                                            int32_t* __restrict__ exps) {
  const int64_t row = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= R) return;
  const uint16_t* xr = x + row * ldx;
  const uint4* src = reinterpret_cast<const uint4*>(xr);
  uint4* dst = reinterpret_cast<uint4*>(y + row * ldy);
  const int K8 = K >> 3;
  int p;
  if (K8 <= kWave * kRegChunks) {
    // the row stays in registers between its reduction and its conversion (one
    // read of x)
    uint4 v[kRegChunks];
    load_row_regs(src, K8, lane, v);
    p = pow2_exp(row_amax_regs(v, K8, lane, l1 != 0), t);
    const float s = pow2f(p);
#pragma unroll
    for (int c = 0; c < kRegChunks; ++c)
      if (lane + c * kWave < K8) dst[lane + c * kWave] = cvt_bf16x8_f16x8(v[c], s);
  } else {
    p = pow2_exp(row_amax_wave(xr, K, lane, l1 != 0), t);
    const float s = pow2f(p);
    for (int i = lane; i < K8; i += kWave) dst[i] = cvt_bf16x8_f16x8(src[i], s);
  }
  if (lane == 0) {
    s_inv[row] = ldexp1(-p);
    if (exps) exps[row] = p;
  }
}

// Transposing convert: yT[c][r] = fp16((x[r][c] * rowmul[r]) * colmul[c]). Each
// thread converts an 8 x 8 block (eight 16-byte row loads) and transposes it in
// registers with v_perm_b32 into eight 16-byte column stores; lane l of a wave
// takes rows 8 (l % 8) and columns 8 (l / 8) of the wave's 64 x 64 square, so
// every load and every store instruction moves whole 128-byte segments and no
// LDS is involved. A block of four waves covers 64 rows x 256 columns. Rows in
// [R, ldyT) are written as zeros, so that the transposed operand can be consumed with a padded contraction length.
// rowmul = 2^rexp[r] or rm[r] (fp32) or 1; colmul = 2^cexp[c] or 1.
__global__ __launch_bounds__(256) void transpose_convert_kernel(const uint16_t* __restrict__ x, int64_t R, int64_t K,
                                                                int64_t ldx, const int32_t* __restrict__ rexp,
                                                                const float* __restrict__ rm,
                                                                const int32_t* __restrict__ cexp,
                                                                uint16_t* __restrict__ yT, int64_t ldyT) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.y * 64 + 8 * (lane & 7);
  const int64_t c0 = (int64_t)blockIdx.x * 256 + 64 * wave + 8 * (lane >> 3);
  if (c0 >= K || r0 >= ldyT) return;
  // all eight loads go out before any is used; rows >= R read row R - 1 and are
  // written as zeros
  uint4 v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = R > 0 ? ldg16(x + min(r0 + i, R - 1) * ldx + c0) : make_uint4(0, 0, 0, 0);
  float cm[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) cm[j] = cexp ? pow2f(cexp[c0 + j]) : 1.f;
  uint32_t w[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t r = min(r0 + i, R - 1);
    const float rmul = R <= 0 ? 0.f : rexp ? pow2f(rexp[r]) : (rm ? rm[r] : 1.f);
    w[i][0] = pack_f16((bf16_lo(v[i].x) * rmul) * cm[0], (bf16_hi(v[i].x) * rmul) * cm[1]);
    w[i][1] = pack_f16((bf16_lo(v[i].y) * rmul) * cm[2], (bf16_hi(v[i].y) * rmul) * cm[3]);
    w[i][2] = pack_f16((bf16_lo(v[i].z) * rmul) * cm[4], (bf16_hi(v[i].z) * rmul) * cm[5]);
    w[i][3] = pack_f16((bf16_lo(v[i].w) * rmul) * cm[6], (bf16_hi(v[i].w) * rmul) * cm[7]);
    if (r0 + i >= R) w[i][0] = w[i][1] = w[i][2] = w[i][3] = 0u;
  }
  // column j: dword k = (row 2k, row 2k + 1) of half j of the rows' dword j / 2
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    const int d = j >> 1;
    stg16(yT + (c0 + j) * ldyT + r0,
          make_uint4(__builtin_amdgcn_perm(w[1][d], w[0][d], sel), __builtin_amdgcn_perm(w[3][d], w[2][d], sel),
                     __builtin_amdgcn_perm(w[5][d], w[4][d], sel), __builtin_amdgcn_perm(w[7][d], w[6][d], sel)));
  }
}

// Column amax partials: each thread covers 8 adjacent columns over a chunk of
// rows; partial[chunk][col] (small_kernels.cu:136-155 merges with atomicMax; the
// partials keep this pass free of a zero-fill and of atomics).
__global__ __launch_bounds__(256) void col_amax_partial_kernel(const uint16_t* __restrict__ x, const float* __restrict__ rm,
                                                               int64_t R, int64_t K, int64_t ldx, int64_t rows_per_chunk,
                                                               float* __restrict__ partial) {
  const int64_t c8 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c8 * 8 >= K) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_chunk;
  const int64_t r1 = min(R, r0 + rows_per_chunk);
  float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll 4
  for (int64_t r = r0; r < r1; ++r) {
    const uint4 v = ldg16(x + r * ldx + c8 * 8);
    const float f = rm ? fabsf(rm[r]) : 1.f;
    m[0] = fmaxf(m[0], fabsf(bf16_lo(v.x)) * f);
    m[1] = fmaxf(m[1], fabsf(bf16_hi(v.x)) * f);
    m[2] = fmaxf(m[2], fabsf(bf16_lo(v.y)) * f);
    m[3] = fmaxf(m[3], fabsf(bf16_hi(v.y)) * f);
    m[4] = fmaxf(m[4], fabsf(bf16_lo(v.z)) * f);
    m[5] = fmaxf(m[5], fabsf(bf16_hi(v.z)) * f);
    m[6] = fmaxf(m[6], fabsf(bf16_lo(v.w)) * f);
    m[7] = fmaxf(m[7], fabsf(bf16_hi(v.w)) * f);
  }
  float* out = partial + (int64_t)blockIdx.y * K + c8 * 8;
  reinterpret_cast<float4*>(out)[0] = make_float4(m[0], m[1], m[2], m[3]);
  reinterpret_cast<float4*>(out)[1] = make_float4(m[4], m[5], m[6], m[7]);
}

// Reduce the partials of each column, then p[c] and s_inv[c] (small_kernels.cu:172,181).
// Block = 64 columns x 4 chunk groups (thread g = tid / 64 takes chunks g, g + 4,
// ... with several loads in flight); the 4 group maxima meet in LDS.
__global__ __launch_bounds__(256) void col_exps_kernel(const float* __restrict__ partial, int64_t nchunks, int64_t K,
                                                       int t, int32_t* __restrict__ cexp, float* __restrict__ s_inv) {
  __shared__ float red[4][64];
  const int cl = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + cl;
  float m = 0.f;
  if (c < K) {
#pragma unroll 8
    for (int64_t i = g; i < nchunks; i += 4) m = fmaxf(m, partial[i * K + c]);
  }
  red[g][cl] = m;
  __syncthreads();
  if (g == 0 && c < K) {
    m = fmaxf(fmaxf(red[0][cl], red[1][cl]), fmaxf(red[2][cl], red[3][cl]));
    const int p = pow2_exp(m, t);
    cexp[c] = p;
    s_inv[c] = ldexp1(-p);
  }
}

__global__ void fill_kernel(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---- attention helpers --------------------------------------------------------

// Per-(b, h) partial maxima of |x| over a chunk of rows: partial[bh * nchunks + chunk].
template <typename T>
__device__ __forceinline__ float amax8(uint4 v);
template <>
__device__ __forceinline__ float amax8<uint16_t>(uint4 v) {  // bf16
  return fmaxf(fmaxf(fmaxf(fabsf(bf16_lo(v.x)), fabsf(bf16_hi(v.x))), fmaxf(fabsf(bf16_lo(v.y)), fabsf(bf16_hi(v.y)))),
               fmaxf(fmaxf(fabsf(bf16_lo(v.z)), fabsf(bf16_hi(v.z))), fmaxf(fabsf(bf16_lo(v.w)), fabsf(bf16_hi(v.w)))));
}
template <>
__device__ __forceinline__ float amax8<_Float16>(uint4 v) {  // fp16
  return fmaxf(fmaxf(fmaxf(fabsf(f16_lo(v.x)), fabsf(f16_hi(v.x))), fmaxf(fabsf(f16_lo(v.y)), fabsf(f16_hi(v.y)))),
               fmaxf(fmaxf(fabsf(f16_lo(v.z)), fabsf(f16_hi(v.z))), fmaxf(fabsf(f16_lo(v.w)), fabsf(f16_hi(v.w)))));
}

// max |x| over rows [chunk * rows_per_chunk, ...) of head (b, h) of a (B, H, S, D)
// tensor, block-wide, into partial[bh * nchunks + chunk]
template <typename T>
__device__ __forceinline__ void head_amax_block(const uint16_t* __restrict__ x, int64_t bh, int64_t H, int64_t S,
                                                int64_t D, int64_t sb, int64_t sh, int64_t ss, int64_t rows_per_chunk,
                                                int64_t nchunks, int64_t chunk, float* __restrict__ partial) {
  const int64_t b = bh / H, h = bh % H;
  const int64_t s0 = chunk * rows_per_chunk, s1 = min(S, s0 + rows_per_chunk);
  const uint16_t* base = x + b * sb + h * sh + s0 * ss;
  const int D8 = (int)(D >> 3), n = (int)((s1 - s0) * D8);
  // eight loads in flight per thread before any of them is reduced
  float m0 = 0.f, m1 = 0.f;
  int i = threadIdx.x;
  for (; i + 7 * 256 < n; i += 8 * 256) {
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int ij = i + j * 256;
      v[j] = ldg16(base + (int64_t)(ij / D8) * ss + (ij % D8) * 8);
    }
    m0 = fmaxf(m0, fmaxf(fmaxf(amax8<T>(v[0]), amax8<T>(v[1])), fmaxf(amax8<T>(v[2]), amax8<T>(v[3]))));
    m1 = fmaxf(m1, fmaxf(fmaxf(amax8<T>(v[4]), amax8<T>(v[5])), fmaxf(amax8<T>(v[6]), amax8<T>(v[7]))));
  }
  for (; i < n; i += 256) m0 = fmaxf(m0, amax8<T>(ldg16(base + (int64_t)(i / D8) * ss + (i % D8) * 8)));
  float m = fmaxf(m0, m1);
  __shared__ float red[4];
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) partial[bh * nchunks + chunk] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <typename T>
__global__ __launch_bounds__(256) void head_amax_partial_kernel(const uint16_t* __restrict__ x, int64_t H, int64_t S,
                                                                int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                                                int64_t rows_per_chunk, int64_t nchunks,
                                                                float* __restrict__ partial) {
  head_amax_block<T>(x, blockIdx.x, H, S, D, sb, sh, ss, rows_per_chunk, nchunks, blockIdx.y, partial);
}

// The same for up to three bf16 tensors in one launch: block x runs over the
// tensors' heads end to end, block y over chunks (past a tensor's own count the
// block has nothing to do).
__global__ __launch_bounds__(256) void head_amax3_kernel(AmaxSegs segs, int64_t D) {
  int64_t bh = blockIdx.x;
  int s = 0;
  while (s + 1 < segs.n && bh >= segs.seg[s].BH) bh -= segs.seg[s++].BH;
  const AmaxSeg& g = segs.seg[s];
  if ((int64_t)blockIdx.y >= g.nch) return;
  head_amax_block<uint16_t>(g.x, bh, g.H, g.S, D, g.sb, g.sh, g.ss, g.rows, g.nch, blockIdx.y, g.partial);
}

__global__ void reduce_partials_kernel(const float* __restrict__ partial, int64_t n, int64_t nchunks,
                                       float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float m = 0.f;
  for (int64_t c = 0; c < nchunks; ++c) m = fmaxf(m, partial[i * nchunks + c]);
  out[i] = m;
}

template <typename Tin, typename Tout>
__device__ __forceinline__ uint4 scale_cast8(uint4 v, float sc);
template <>
__device__ __forceinline__ uint4 scale_cast8<uint16_t, _Float16>(uint4 v, float sc) {
  return cvt_bf16x8_f16x8(v, sc);
}
template <>
__device__ __forceinline__ uint4 scale_cast8<uint16_t, uint16_t>(uint4 v, float sc) {
  return make_uint4(pack_bf16(bf16_lo(v.x) * sc, bf16_hi(v.x) * sc), pack_bf16(bf16_lo(v.y) * sc, bf16_hi(v.y) * sc),
                    pack_bf16(bf16_lo(v.z) * sc, bf16_hi(v.z) * sc), pack_bf16(bf16_lo(v.w) * sc, bf16_hi(v.w) * sc));
}
template <>
__device__ __forceinline__ uint4 scale_cast8<_Float16, uint16_t>(uint4 v, float sc) {
  return make_uint4(pack_bf16(f16_lo(v.x) * sc, f16_hi(v.x) * sc), pack_bf16(f16_lo(v.y) * sc, f16_hi(v.y) * sc),
                    pack_bf16(f16_lo(v.z) * sc, f16_hi(v.z) * sc), pack_bf16(f16_lo(v.w) * sc, f16_hi(v.w) * sc));
}
template <>
__device__ __forceinline__ uint4 scale_cast8<_Float16, _Float16>(uint4 v, float sc) {
  return make_uint4(pack_f16(f16_lo(v.x) * sc, f16_hi(v.x) * sc), pack_f16(f16_lo(v.y) * sc, f16_hi(v.y) * sc),
                    pack_f16(f16_lo(v.z) * sc, f16_hi(v.z) * sc), pack_f16(f16_lo(v.w) * sc, f16_hi(v.w) * sc));
}

// y (contiguous) = x * 2^e[b, h] (small_kernels.cu:246-263). The scale is built
// with ldexp so any int32 exponent that keeps the result representable works.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(256) void head_scale_cast_kernel(const uint16_t* __restrict__ x, int64_t H, int64_t S,
                                                              int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                                              const int32_t* __restrict__ e, int64_t e_sb,
                                                              int64_t e_sh, uint16_t* __restrict__ y, int64_t total8) {
  const int64_t D8 = D >> 3;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total8; i += (int64_t)gridDim.x * 256) {
    const int64_t d = (i % D8) * 8, row = i / D8, s = row % S, bh = row / S, b = bh / H, h = bh % H;
    const float sc = ldexp1(e[b * e_sb + h * e_sh]);
    stg16(y + i * 8, scale_cast8<Tin, Tout>(ldg16(x + b * sb + h * sh + s * ss + d), sc));
  }
}

// M = 1 GEMV (small_kernels.cu:107-132): one wave per output, fp32 FMA on bf16 x
// and fp16 w, no activation scale.
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                   const float* __restrict__ ws, const uint16_t* __restrict__ bias,
                                                   uint16_t* __restrict__ y, int64_t N, int K, int64_t ldw) {
  const int64_t n = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const uint4* xr = reinterpret_cast<const uint4*>(x);
  const uint4* wr = reinterpret_cast<const uint4*>(w + n * ldw);
  float a0 = 0.f, a1 = 0.f;
  const int K8 = K >> 3;
  // UG chunks of 16 bytes per lane per round, all loads issued before the FMAs:
  // the weight stream needs several loads in flight per lane to approach HBM
  // bandwidth (one per iteration had held it at ~4.2 TB/s)
  constexpr int UG = 8;
  for (int base = 0; base < K8; base += UG * kWave) {
    uint4 xv[UG], wv[UG];
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const int i = base + u * kWave + lane;
      xv[u] = i < K8 ? xr[i] : make_uint4(0, 0, 0, 0);
      wv[u] = i < K8 ? wr[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      a0 = fmaf(bf16_lo(xv[u].x), f16_lo(wv[u].x), a0);
      a1 = fmaf(bf16_hi(xv[u].x), f16_hi(wv[u].x), a1);
      a0 = fmaf(bf16_lo(xv[u].y), f16_lo(wv[u].y), a0);
      a1 = fmaf(bf16_hi(xv[u].y), f16_hi(wv[u].y), a1);
      a0 = fmaf(bf16_lo(xv[u].z), f16_lo(wv[u].z), a0);
      a1 = fmaf(bf16_hi(xv[u].z), f16_hi(wv[u].z), a1);
      a0 = fmaf(bf16_lo(xv[u].w), f16_lo(wv[u].w), a0);
      a1 = fmaf(bf16_hi(xv[u].w), f16_hi(wv[u].w), a1);
    }
  }
  const float acc = wave_sum(a0 + a1);
  if (lane == 0) {
    float r = acc * ws[n];
    if (bias) r += bf16_lo(bias[n]);
    const uint32_t packed = pack_bf16(r, 0.f);
    y[n] = (uint16_t)(packed & 0xffffu);
  }
}

int check_rows(const char* fn, const void* x, int64_t R, int64_t K, int64_t ldx) {
  TB_CHECK(x != nullptr || R * K == 0, "%s: null input", fn);
  TB_CHECK(R >= 0 && K >= 0, "%s: negative shape", fn);
  TB_CHECK(K % 8 == 0 && ldx % 8 == 0 && ldx >= K && aligned16(x),
           "%s: K and row stride must be multiples of 8", fn);
  TB_CHECK(K < (int64_t)1 << 31, "%s: K too large", fn);
  return 0;
}

int64_t col_chunks(int64_t R, int64_t K) {
  const int64_t col_blocks = cdiv(cdiv(K, 8), 256);
  int64_t chunks = cdiv(1024, col_blocks);
  chunks = std::max<int64_t>(1, std::min<int64_t>(chunks, cdiv(R, 32)));
  return chunks;
}

// ~512 blocks per tensor of at least 64 rows each: 32 KB a block at D = 128 (eight
// 16-byte loads per thread), and few partials for the exponent derivation that
// every block of the attention's conversion pass repeats
int64_t head_chunks(int64_t BH, int64_t S) {
  return std::max<int64_t>(1, std::min<int64_t>(cdiv(512, std::max<int64_t>(BH, 1)), cdiv(S, 64)));
}

}  // namespace

// Shared with attention.hip: partial head maxima in one launch per tensor.
namespace tbf16 {
int64_t head_amax_chunks(int64_t BH, int64_t S) { return head_chunks(BH, S); }

int launch_head_amax3(const AmaxSegs& segs, int64_t D, hipStream_t st) {
  int64_t bhs = 0, nch = 0;
  for (int i = 0; i < segs.n; ++i) {
    bhs += segs.seg[i].BH;
    nch = std::max(nch, segs.seg[i].nch);
  }
  if (bhs == 0) return 0;
  head_amax3_kernel<<<dim3((unsigned)bhs, (unsigned)nch), 256, 0, st>>>(segs, D);
  TB_LAUNCH_CHECK("head_amax3");
  return 0;
}

int launch_head_amax_partial(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                             int64_t sh, int64_t ss, float* partial, int64_t nchunks, hipStream_t st) {
  const int64_t rows = cdiv(S, nchunks);
  dim3 grid((unsigned)(B * H), (unsigned)nchunks);
  if (dtype == TBF16_DT_BF16)
    head_amax_partial_kernel<uint16_t><<<grid, 256, 0, st>>>((const uint16_t*)x, H, S, D, sb, sh, ss, rows, nchunks,
                                                             partial);
  else
    head_amax_partial_kernel<_Float16><<<grid, 256, 0, st>>>((const uint16_t*)x, H, S, D, sb, sh, ss, rows, nchunks,
                                                             partial);
  TB_LAUNCH_CHECK("head_amax");
  return 0;
}

int launch_row_exps(const void* x, int64_t M, int64_t K, int64_t ldx, int t, int l1, int32_t* exps, float* s_inv,
                    hipStream_t st) {
  if (M == 0) return 0;
  row_exps_kernel<<<(unsigned)cdiv(M, kRowWaves), 256, 0, st>>>((const uint16_t*)x, M, (int)K, ldx, t, l1, exps, s_inv);
  TB_LAUNCH_CHECK("row_exps");
  return 0;
}

// y16 = fp16(x * 2^p[r]), s_inv[r] = 2^-p[r] and, if exps is given, exps[r] = p[r]
int launch_quantize_rows(const void* x, int64_t R, int64_t K, int64_t ldx, int t, int l1, void* y16, int64_t ldy,
                         float* s_inv, int32_t* exps, hipStream_t st) {
  if (R == 0) return 0;
  quantize_rows_kernel<<<(unsigned)cdiv(R, kRowWaves), 256, 0, st>>>((const uint16_t*)x, R, (int)K, ldx, t, l1,
                                                                     (uint16_t*)y16, ldy, s_inv, exps);
  TB_LAUNCH_CHECK("quantize_rows");
  return 0;
}
}  // namespace tbf16

extern "C" int tbf16_row_exps(const void* x, int64_t M, int64_t K, int64_t ldx, int t, int l1, int32_t* exps,
                              float* s_inv, void* stream) {
  if (int rc = check_rows("row_exps", x, M, K, ldx)) return rc;
  TB_CHECK(exps != nullptr || s_inv != nullptr, "row_exps: no output");
  return launch_row_exps(x, M, K, ldx, t, l1, exps, s_inv, as_stream(stream));
}

extern "C" int tbf16_quantize_rows(const void* x, int64_t R, int64_t K, int64_t ldx, int t, int l1, void* y16,
                                   int64_t ldy, float* s_inv, void* stream) {
  if (int rc = check_rows("quantize_rows", x, R, K, ldx)) return rc;
  TB_CHECK(ldy % 8 == 0 && ldy >= K && aligned16(y16) && s_inv, "quantize_rows: bad output");
  if (R == 0) return 0;
  return launch_quantize_rows(x, R, K, ldx, t, l1, y16, ldy, s_inv, nullptr, as_stream(stream));
}

extern "C" int tbf16_quantize_rows_t(const void* x, int64_t R, int64_t K, int64_t ldx, int t, void* yT, int64_t ldyT,
                                     float* s_inv, int32_t* exps_ws, void* stream) {
  if (int rc = check_rows("quantize_rows_t", x, R, K, ldx)) return rc;
  TB_CHECK(ldyT % 8 == 0 && ldyT >= R && aligned16(yT) && s_inv && exps_ws, "quantize_rows_t: bad output");
  hipStream_t st = as_stream(stream);
  if (R > 0) {
    if (int rc = launch_row_exps(x, R, K, ldx, t, 0, exps_ws, s_inv, st)) return rc;
  }
  if (K == 0 || ldyT == 0) return 0;
  dim3 grid((unsigned)cdiv(K, 256), (unsigned)cdiv(ldyT, 64));
  transpose_convert_kernel<<<grid, 256, 0, st>>>((const uint16_t*)x, R, K, ldx, exps_ws, nullptr, nullptr,
                                                 (uint16_t*)yT, ldyT);
  TB_LAUNCH_CHECK("quantize_rows_t");
  return 0;
}

extern "C" size_t tbf16_quantize_cols_ws_bytes(int64_t R, int64_t K) {
  const int64_t ch = col_chunks(R, K);
  return align_up((size_t)(ch * K) * sizeof(float), 256) + align_up((size_t)K * sizeof(int32_t), 256);
}

extern "C" int tbf16_quantize_cols_t(const void* x, int64_t R, int64_t K, int64_t ldx, int t, const float* row_mul,
                                     void* yT, int64_t ldyT, float* s_inv, void* ws, int64_t ws_bytes, void* stream) {
  if (int rc = check_rows("quantize_cols", x, R, K, ldx)) return rc;
  TB_CHECK(ldyT % 8 == 0 && ldyT >= R && aligned16(yT) && s_inv, "quantize_cols: bad output");
  TB_CHECK(ws != nullptr && ws_bytes >= (int64_t)tbf16_quantize_cols_ws_bytes(R, K), "quantize_cols: workspace too small");
  hipStream_t st = as_stream(stream);
  if (K == 0) return 0;
  const int64_t ch = col_chunks(R, K);
  float* partial = reinterpret_cast<float*>(ws);
  int32_t* cexp = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(ws) + align_up((size_t)(ch * K) * sizeof(float), 256));
  if (R > 0) {
    dim3 g1((unsigned)cdiv(cdiv(K, 8), 256), (unsigned)ch);
    col_amax_partial_kernel<<<g1, 256, 0, st>>>((const uint16_t*)x, row_mul, R, K, ldx, cdiv(R, ch), partial);
    TB_LAUNCH_CHECK("quantize_cols/amax");
    col_exps_kernel<<<(unsigned)cdiv(K, 64), 256, 0, st>>>(partial, ch, K, t, cexp, s_inv);
    TB_LAUNCH_CHECK("quantize_cols/exps");
  } else {  // no rows: s_inv = 1 as the reference returns (small_kernels.cu:325)
    fill_kernel<<<(unsigned)cdiv(K, 256), 256, 0, st>>>(s_inv, K, 1.0f);
    TB_LAUNCH_CHECK("quantize_cols/fill");
  }
  if (ldyT == 0) return 0;
  dim3 grid((unsigned)cdiv(K, 256), (unsigned)cdiv(ldyT, 64));
  transpose_convert_kernel<<<grid, 256, 0, st>>>((const uint16_t*)x, R, K, ldx, nullptr, row_mul, cexp, (uint16_t*)yT,
                                                 ldyT);
  TB_LAUNCH_CHECK("quantize_cols/convert");
  return 0;
}

extern "C" int tbf16_gemv(const void* x, const void* w16, int64_t N, int64_t K, int64_t ldw, const float* ws,
                          const void* bias, void* y, void* stream) {
  TB_CHECK(K % 8 == 0 && ldw % 8 == 0 && ldw >= K && aligned16(x) && aligned16(w16), "gemv: K and row stride must be multiples of 8");
  TB_CHECK(ws && y, "gemv: bad arguments");
  if (N == 0) return 0;
  gemv_kernel<<<(unsigned)cdiv(N, kRowWaves), 256, 0, as_stream(stream)>>>(
      (const uint16_t*)x, (const uint16_t*)w16, ws, (const uint16_t*)bias, (uint16_t*)y, N, (int)K, ldw);
  TB_LAUNCH_CHECK("gemv");
  return 0;
}

extern "C" int tbf16_head_amax(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                               int64_t sh, int64_t ss, float* out, void* stream) {
  TB_CHECK(dtype == TBF16_DT_BF16 || dtype == TBF16_DT_F16, "head_amax: bf16 or fp16");
  TB_CHECK(D % 8 == 0 && sb % 8 == 0 && sh % 8 == 0 && ss % 8 == 0 && aligned16(x),
           "expected (B, H, S, D) with contiguous D %% 8 == 0");
  TB_CHECK(out != nullptr, "head_amax: null output");
  const int64_t BH = B * H;
  if (BH == 0) return 0;
  hipStream_t st = as_stream(stream);
  TB_CHECK(S > 0 && D > 0, "head_amax: empty heads are handled by the caller");
  // One block per head writes its maximum straight into out (no partials, no
  // zero-fill). The fused attention path uses the chunked partial launch instead.
  const int64_t nchunks = 1;
  const int64_t rows = S;
  dim3 grid((unsigned)BH, (unsigned)nchunks);
  if (dtype == TBF16_DT_BF16)
    head_amax_partial_kernel<uint16_t><<<grid, 256, 0, st>>>((const uint16_t*)x, H, S, D, sb, sh, ss, rows, nchunks, out);
  else
    head_amax_partial_kernel<_Float16><<<grid, 256, 0, st>>>((const uint16_t*)x, H, S, D, sb, sh, ss, rows, nchunks, out);
  TB_LAUNCH_CHECK("head_amax");
  return 0;
}

extern "C" int tbf16_head_scale_cast(const void* x, int in_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                     int64_t sb, int64_t sh, int64_t ss, const int32_t* e, int64_t e_sb, int64_t e_sh,
                                     void* y, int out_dtype, void* stream) {
  TB_CHECK((in_dtype == TBF16_DT_BF16 || in_dtype == TBF16_DT_F16) &&
               (out_dtype == TBF16_DT_BF16 || out_dtype == TBF16_DT_F16),
           "head_scale_cast: bf16/fp16 only");
  TB_CHECK(D % 8 == 0 && sb % 8 == 0 && sh % 8 == 0 && ss % 8 == 0 && aligned16(x) && aligned16(y),
           "expected (B, H, S, D) with contiguous D %% 8 == 0");
  const int64_t total8 = B * H * S * D / 8;
  if (total8 == 0) return 0;
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(total8, 256), 256 * 16);
  hipStream_t st = as_stream(stream);
#define LAUNCH(TI, TO)                                                                                           \
  head_scale_cast_kernel<TI, TO><<<blocks, 256, 0, st>>>((const uint16_t*)x, H, S, D, sb, sh, ss, e, e_sb, e_sh, \
                                                         (uint16_t*)y, total8)
  if (in_dtype == TBF16_DT_BF16 && out_dtype == TBF16_DT_F16) LAUNCH(uint16_t, _Float16);
  else if (in_dtype == TBF16_DT_F16 && out_dtype == TBF16_DT_BF16) LAUNCH(_Float16, uint16_t);
  else if (in_dtype == TBF16_DT_BF16) LAUNCH(uint16_t, uint16_t);
  else LAUNCH(_Float16, _Float16);
#undef LAUNCH
  TB_LAUNCH_CHECK("head_scale_cast");
  return 0;
}
