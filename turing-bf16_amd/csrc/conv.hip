// Scaled convolutions (tbf16/conv.py of the reference): a bf16 convolution runs
// as an fp16 one on inputs scaled by exact powers of two -- one exponent per
// sample for the input (a convolution mixes positions, so rows cannot be scaled
// separately) and one per output channel for the weight -- and the scales are
// undone in an epilogue that writes bf16. The fp16 convolution itself is
// MIOpen's (called by the Python layer); these kernels are the passes around it.
//
// Memory layout: a sample is n = C * prod(spatial) elements stored back to back
// (contiguous NC... or channels-last, both keep the batch outermost), so the
// input passes run over B * n elements in memory order and find the sample as
// index / n. All three kernels are HBM-bound streams of 16-byte vectors.
#include <algorithm>

#include "abi_util.h"
#include "common.h"

namespace {
using namespace tbf16;

constexpr int kThreads = 256;
// Elements of one sample per block of the input passes (a multiple of 8).
constexpr int64_t kChunk = 8192;

__device__ __forceinline__ uint32_t mag_max2(uint32_t w, uint32_t m) {
  return max(m, max(w & 0x7FFFu, (w >> 16) & 0x7FFFu));
}

// Largest bf16 magnitude as its bit pattern. An unsigned max of |x| bits orders
// finite values as their magnitudes, puts inf above them and every NaN pattern
// above inf, so one NaN makes the maximum NaN, as torch's max-norm does.
__device__ __forceinline__ uint32_t mag_max8(uint4 v, uint32_t m) {
  return mag_max2(v.w, mag_max2(v.z, mag_max2(v.y, mag_max2(v.x, m))));
}

// Exponent of the per-sample scale (conv.py:28-31,49-50): frexp(amax) - t, with
// all-zero and NaN samples taken as amax = 1 (torch.where(amax > 0, amax, 1)) and
// inf giving frexp's 0.
__device__ __forceinline__ int sample_exp(uint32_t m, int t) {
  if (m == 0u || m > 0x7F80u) return 1 - t;
  return frexp_exp(__uint_as_float(m << 16)) - t;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t m) {
  __shared__ uint32_t red[kThreads / kWave];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, kWave));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / kWave; ++w) r = max(r, red[w]);
  return r;
}

// Elements [lo, hi) of x: scalar reads for the unaligned ends, 16-byte vectors
// (x is 16-byte aligned at element 0, so vectors sit at multiples of 8
// elements) with four loads in flight per lane for the rest. f(v, vec) takes
// each vector with its index, g(i) each scalar element.
template <typename FV, typename FS>
__device__ __forceinline__ void for_run(int64_t lo, int64_t hi, FV f, FS g) {
  const int64_t vlo = (lo + 7) >> 3, vhi = hi >> 3;
  if (vlo >= vhi) {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) g(i);
    return;
  }
  for (int64_t i = lo + threadIdx.x; i < vlo * 8; i += kThreads) g(i);
  for (int64_t i = vhi * 8 + threadIdx.x; i < hi; i += kThreads) g(i);
  int64_t v = vlo + threadIdx.x;
  for (; v + 3 * kThreads < vhi; v += 4 * kThreads) f(v, 4);
  for (; v < vhi; v += kThreads) f(v, 1);
}

// Block b * nch + c reduces elements [c * kChunk, (c + 1) * kChunk) of sample b
// into partial[b * nch + c].
__global__ __launch_bounds__(kThreads) void sample_amax_kernel(const uint16_t* __restrict__ x, int64_t n, int nch,
                                                               uint32_t* __restrict__ partial) {
  const int64_t b = blockIdx.x / nch;
  const int64_t c = blockIdx.x - b * nch;
  const int64_t lo = b * n + c * kChunk;
  const int64_t hi = std::min(b * n + n, lo + kChunk);
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  uint32_t m = 0u;
  for_run(
      lo, hi,
      [&](int64_t v, int cnt) {
        if (cnt == 4) {
          const uint4 a0 = xv[v], a1 = xv[v + kThreads], a2 = xv[v + 2 * kThreads], a3 = xv[v + 3 * kThreads];
          m = mag_max8(a3, mag_max8(a2, mag_max8(a1, mag_max8(a0, m))));
        } else {
          m = mag_max8(xv[v], m);
        }
      },
      [&](int64_t i) { m = max(m, x[i] & 0x7FFFu); });
  m = block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// Block b * nch + c: the exponent of sample b from its nch partial maxima, then
// x16 = fp16(x * 2^-e) for the same elements the max pass block covered
// (conv.py:51-54: torch.mul of bf16 by the fp32 scale ldexp(1, -e), written to
// fp16: one RNE rounding of the fp32 product). The scale is ldexp(1, -e) in
// fp32, so -e >= 128 gives inf exactly as the reference does.
__global__ __launch_bounds__(kThreads) void sample_cast_kernel(const uint16_t* __restrict__ x, int64_t n, int nch,
                                                               const uint32_t* __restrict__ partial, int t,
                                                               int32_t* __restrict__ exps,
                                                               uint16_t* __restrict__ y) {
  const int64_t b = blockIdx.x / nch;
  const int64_t c = blockIdx.x - b * nch;
  uint32_t m = 0u;
  for (int i = threadIdx.x; i < nch; i += kThreads) m = max(m, partial[b * nch + i]);
  const int e = sample_exp(block_max_u32(m), t);
  if (c == 0 && threadIdx.x == 0) exps[b] = e;
  const float s = ldexp1(-e);
  const int64_t lo = b * n + c * kChunk;
  const int64_t hi = std::min(b * n + n, lo + kChunk);
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  uint4* yv = reinterpret_cast<uint4*>(y);
  for_run(
      lo, hi,
      [&](int64_t v, int cnt) {
        if (cnt == 4) {
          const uint4 a0 = xv[v], a1 = xv[v + kThreads], a2 = xv[v + 2 * kThreads], a3 = xv[v + 3 * kThreads];
          yv[v] = cvt_bf16x8_f16x8(a0, s);
          yv[v + kThreads] = cvt_bf16x8_f16x8(a1, s);
          yv[v + 2 * kThreads] = cvt_bf16x8_f16x8(a2, s);
          yv[v + 3 * kThreads] = cvt_bf16x8_f16x8(a3, s);
        } else {
          yv[v] = cvt_bf16x8_f16x8(xv[v], s);
        }
      },
      [&](int64_t i) { y[i] = __builtin_bit_cast(uint16_t, (_Float16)(__uint_as_float((uint32_t)x[i] << 16) * s)); });
}

// out = bf16(y * (2^exps[b] * ws[o]) [+ bias[o]]) in fp32 (conv.py:56-60): the
// scale is the fp32 product of the two powers of two, y * scale is exact unless
// it leaves fp32's normal range, the bias add rounds once to fp32 and the result
// once more to bf16, as torch's mul / addcmul into a bf16 tensor do.
// CL = 0: (B, O, P) layout, CL = 1: (B, P, O).
template <bool BIAS>
__device__ __forceinline__ float epi_elem(float v, float sc, float bias) {
  return BIAS ? fmaf(v, sc, bias) : v * sc;
}

// ALIGNED: every 16-byte vector lies in one (b, o) row (CL = 0, P % 8 == 0) or
// covers 8 channels of one pixel starting at a multiple of 8 (CL = 1, O % 8 == 0,
// ws and bias 16-byte aligned), so the scales are found once per vector.
template <bool CL, bool BIAS, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void conv_epilogue_kernel(const uint16_t* __restrict__ y, int64_t O, int64_t P,
                                                                 int64_t total, const int32_t* __restrict__ exps,
                                                                 const float* __restrict__ ws,
                                                                 const float* __restrict__ bias,
                                                                 uint16_t* __restrict__ out) {
  const int64_t nv = total >> 3;
  for (int64_t v = (int64_t)blockIdx.x * kThreads + threadIdx.x; v < nv; v += (int64_t)gridDim.x * kThreads) {
    const int64_t i0 = v * 8;
    const uint4 in = reinterpret_cast<const uint4*>(y)[v];
    const uint32_t w[4] = {in.x, in.y, in.z, in.w};
    float r[8];
    if constexpr (ALIGNED && !CL) {
      const int64_t row = i0 / P, b = row / O, o = row - b * O;
      const float sc = ldexp1(exps[b]) * ws[o], bs = BIAS ? bias[o] : 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = epi_elem<BIAS>((k & 1) ? f16_hi(w[k >> 1]) : f16_lo(w[k >> 1]), sc, bs);
    } else if constexpr (ALIGNED) {
      const int64_t q = i0 / O, o = i0 - q * O, b = q / P;
      const float eb = ldexp1(exps[b]);
      const float4 w0 = *reinterpret_cast<const float4*>(ws + o), w1 = *reinterpret_cast<const float4*>(ws + o + 4);
      float4 b0 = make_float4(0.f, 0.f, 0.f, 0.f), b1 = b0;
      if constexpr (BIAS) {
        b0 = *reinterpret_cast<const float4*>(bias + o);
        b1 = *reinterpret_cast<const float4*>(bias + o + 4);
      }
      const float wk[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      const float bk[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int k = 0; k < 8; ++k)
        r[k] = epi_elem<BIAS>((k & 1) ? f16_hi(w[k >> 1]) : f16_lo(w[k >> 1]), eb * wk[k], bk[k]);
    } else if constexpr (!CL) {
      // elements run along P within one (b, o) row; a row change is rare
      int64_t row = i0 / P, p = i0 - row * P;
      int64_t b = row / O, o = row - b * O;
      float sc = ldexp1(exps[b]) * ws[o], bs = BIAS ? bias[o] : 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        r[k] = epi_elem<BIAS>((k & 1) ? f16_hi(w[k >> 1]) : f16_lo(w[k >> 1]), sc, bs);
        if (k < 7 && ++p == P) {
          p = 0;
          if (++o == O) o = 0, ++b;
          sc = ldexp1(exps[b]) * ws[o];
          if (BIAS) bs = bias[o];
        }
      }
    } else {
      // elements run along O within one pixel
      const int64_t q = i0 / O;
      int64_t o = i0 - q * O;
      int64_t b = q / P, pix = q - b * P;
      float eb = ldexp1(exps[b]);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        r[k] = epi_elem<BIAS>((k & 1) ? f16_hi(w[k >> 1]) : f16_lo(w[k >> 1]), eb * ws[o], BIAS ? bias[o] : 0.f);
        if (k < 7 && ++o == O) {
          o = 0;
          if (++pix == P) pix = 0, ++b, eb = ldexp1(exps[b]);
        }
      }
    }
    reinterpret_cast<uint4*>(out)[v] =
        make_uint4(pack_bf16(r[0], r[1]), pack_bf16(r[2], r[3]), pack_bf16(r[4], r[5]), pack_bf16(r[6], r[7]));
  }
  if (blockIdx.x == 0) {
    for (int64_t i = nv * 8 + threadIdx.x; i < total; i += kThreads) {
      int64_t b, o;
      if constexpr (!CL) {
        const int64_t row = i / P;
        b = row / O;
        o = row - b * O;
      } else {
        o = i % O;
        b = i / O / P;
      }
      const float val = (float)__builtin_bit_cast(_Float16, y[i]);
      const float rr = epi_elem<BIAS>(val, ldexp1(exps[b]) * ws[o], BIAS ? bias[o] : 0.f);
      out[i] = __builtin_bit_cast(uint16_t, (__bf16)rr);
    }
  }
}

int64_t amax_chunks(int64_t n) { return std::max<int64_t>(1, cdiv(n, kChunk)); }

unsigned stream_blocks(int64_t nv) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(nv, kThreads), 4096)); }

}  // namespace

extern "C" size_t tbf16_conv_input_ws_bytes(int64_t B, int64_t n) {
  if (B <= 0 || n <= 0) return 0;
  return align_up((size_t)(B * amax_chunks(n)) * sizeof(uint32_t), 256);
}

extern "C" int tbf16_conv_input(const void* x, int64_t B, int64_t n, int t, int32_t* exps, void* x16, void* ws,
                                int64_t ws_bytes, void* stream) {
  TB_CHECK(B >= 0 && n >= 0, "conv_input: negative size");
  if (B == 0) return 0;
  TB_CHECK(x && exps && x16, "conv_input: null pointer");
  TB_CHECK(aligned16(x) && aligned16(x16), "conv_input: x and x16 must be 16-byte aligned");
  TB_CHECK(n > 0, "conv_input: empty samples are handled by the caller");
  const int64_t nch = amax_chunks(n);
  TB_CHECK(B * nch <= 0x7FFFFFFF, "conv_input: tensor too large");
  TB_CHECK(ws && ws_bytes >= (int64_t)tbf16_conv_input_ws_bytes(B, n), "conv_input: workspace too small");
  hipStream_t st = as_stream(stream);
  sample_amax_kernel<<<(unsigned)(B * nch), kThreads, 0, st>>>((const uint16_t*)x, n, (int)nch, (uint32_t*)ws);
  TB_LAUNCH_CHECK("conv_input (max)");
  sample_cast_kernel<<<(unsigned)(B * nch), kThreads, 0, st>>>((const uint16_t*)x, n, (int)nch, (const uint32_t*)ws,
                                                               t, exps, (uint16_t*)x16);
  TB_LAUNCH_CHECK("conv_input (cast)");
  return 0;
}

extern "C" int tbf16_conv_epilogue(const void* y16, int64_t B, int64_t O, int64_t P, int channels_last,
                                   const int32_t* exps, const float* ws, const float* bias, void* out, void* stream) {
  TB_CHECK(B >= 0 && O >= 0 && P >= 0, "conv_epilogue: negative size");
  const int64_t total = B * O * P;
  if (total == 0) return 0;
  TB_CHECK(y16 && exps && ws && out, "conv_epilogue: null pointer");
  TB_CHECK(aligned16(y16) && aligned16(out), "conv_epilogue: y16 and out must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  const unsigned blocks = stream_blocks(total >> 3);
  const bool aligned = channels_last ? (O % 8 == 0 && aligned16(ws) && (!bias || aligned16(bias))) : P % 8 == 0;
#define LAUNCH(CL, BI, AL)                                                                                    \
  conv_epilogue_kernel<CL, BI, AL><<<blocks, kThreads, 0, st>>>((const uint16_t*)y16, O, P, total, exps, ws, bias, \
                                                                (uint16_t*)out)
#define LAUNCH2(CL, BI) \
  if (aligned) LAUNCH(CL, BI, true); else LAUNCH(CL, BI, false)
  if (channels_last) {
    if (bias) { LAUNCH2(true, true); } else { LAUNCH2(true, false); }
  } else {
    if (bias) { LAUNCH2(false, true); } else { LAUNCH2(false, false); }
  }
#undef LAUNCH2
#undef LAUNCH
  TB_LAUNCH_CHECK("conv_epilogue");
  return 0;
}
