// Shared device helpers for the tbf16 HIP library (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tbf16 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf162v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---- exponent arithmetic -------------------------------------------------

__device__ __forceinline__ int exp_field(float a) { return (__float_as_int(a) >> 23) & 0xFF; }

// Scale exponent p (scale = 2^p) that puts a normal amax in [2^(t-1), 2^t):
// e = clamp(E(amax), 1, 252), se = clamp(253 + t - e, 1, 254), p = se - 127.
// Reference: tbf16/csrc/small_kernels.cu:12-18 (gemm_sm75.cu:19-23 only differs
// for t < 2, which the fused path never uses).
__device__ __forceinline__ int pow2_exp(float amax, int t) {
  int e = min(max(exp_field(amax), 1), 252);
  int se = min(max(253 + t - e, 1), 254);
  return se - 127;
}

// 2^p as an fp32 for p in [-126, 127] (exact, built from exponent bits).
__device__ __forceinline__ float pow2f(int p) { return __int_as_float((p + 127) << 23); }

// 2^p for any p where the result is representable (subnormals included).
__device__ __forceinline__ float ldexp1(int p) { return __builtin_amdgcn_ldexpf(1.0f, p); }

// torch.frexp exponent: x = m * 2^e with m in [0.5, 1); 0 for 0, inf and nan.
__device__ __forceinline__ int frexp_exp(float x) { return __builtin_amdgcn_frexp_expf(x); }

// ---- conversions ------------------------------------------------------------

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Two fp32 -> packed fp16, round to nearest even (v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  half2v h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, h);
}

// Two fp32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf162v h = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ float f16_lo(uint32_t v) {
  return (float)__builtin_bit_cast(half2v, v)[0];
}
__device__ __forceinline__ float f16_hi(uint32_t v) {
  return (float)__builtin_bit_cast(half2v, v)[1];
}

// Packed bf16 pair -> packed fp16 pair scaled by s = 2^p (exact in fp16's normal
// range, RNE for fp16 subnormals), as quantize_rows does (small_kernels.cu:68-69).
__device__ __forceinline__ uint32_t cvt_bf16x2_f16x2(uint32_t v, float s) {
  return pack_f16(bf16_lo(v) * s, bf16_hi(v) * s);
}

__device__ __forceinline__ uint4 cvt_bf16x8_f16x8(uint4 v, float s) {
  return make_uint4(cvt_bf16x2_f16x2(v.x, s), cvt_bf16x2_f16x2(v.y, s), cvt_bf16x2_f16x2(v.z, s),
                    cvt_bf16x2_f16x2(v.w, s));
}

// ---- wave reductions (64 lanes) ----------------------------------------------

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// amax (or L1 norm) of a bf16 row, reduced over the wave; valid in every lane.
// L1 accumulates in fp64 and rounds once to fp32, so the exponent is that of the
// exact sum (the reference's fp32 thread-order sum, small_kernels.cu:42-59, can
// differ only within one fp32 ulp of a power of two).
// L1 sum of one 16-byte chunk (8 bf16) in fp64, left to right; row_amax_regs adds
// its chunks with the same expression.
__device__ __forceinline__ double l1_chunk(uint4 v) {
  return (double)fabsf(bf16_lo(v.x)) + (double)fabsf(bf16_hi(v.x)) + (double)fabsf(bf16_lo(v.y)) +
         (double)fabsf(bf16_hi(v.y)) + (double)fabsf(bf16_lo(v.z)) + (double)fabsf(bf16_hi(v.z)) +
         (double)fabsf(bf16_lo(v.w)) + (double)fabsf(bf16_hi(v.w));
}
__device__ __forceinline__ float max_chunk(uint4 a) {
  return fmaxf(fmaxf(fmaxf(fabsf(bf16_lo(a.x)), fabsf(bf16_hi(a.x))), fmaxf(fabsf(bf16_lo(a.y)), fabsf(bf16_hi(a.y)))),
               fmaxf(fmaxf(fabsf(bf16_lo(a.z)), fabsf(bf16_hi(a.z))), fmaxf(fabsf(bf16_lo(a.w)), fabsf(bf16_hi(a.w)))));
}
// Four chunks' loads are issued before any is used, so a lane has four 16-byte
// loads in flight instead of one (a row of K = 6144 is 12 chunks per lane: one at
// a time, the L1 pass on dY ran at 3.4 TB/s). The L1 sum still adds the chunks in
// the order lane, lane + 64, ... into one accumulator: the same bits as one chunk
// per iteration.
__device__ __forceinline__ float row_amax_wave(const uint16_t* xr, int K, int lane, bool l1) {
  const uint4* p = reinterpret_cast<const uint4*>(xr);
  const int K8 = K >> 3;
  constexpr int U = 4;
  int i = lane;
  if (l1) {
    double acc = 0.0;
    for (; i + (U - 1) * kWave < K8; i += U * kWave) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = p[i + u * kWave];
#pragma unroll
      for (int u = 0; u < U; ++u) acc += l1_chunk(v[u]);
    }
    for (; i < K8; i += kWave) acc += l1_chunk(p[i]);
    return (float)wave_sum_d(acc);
  }
  float m0 = 0.f, m1 = 0.f;
  for (; i + (U - 1) * kWave < K8; i += U * kWave) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = p[i + u * kWave];
    m0 = fmaxf(m0, fmaxf(max_chunk(v[0]), max_chunk(v[2])));
    m1 = fmaxf(m1, fmaxf(max_chunk(v[1]), max_chunk(v[3])));
  }
  for (; i < K8; i += kWave) m0 = fmaxf(m0, max_chunk(p[i]));
  return wave_max(fmaxf(m0, m1));
}

// ---- memory ------------------------------------------------------------------

typedef int int4v __attribute__((ext_vector_type(4)));

// The raw buffer load intrinsic with a 4 x i32 resource (this form keeps the
// descriptor in SGPRs; the pointer-typed builtin lost uniformity through the
// staging lambdas and produced a waterfall loop around every load).
__device__ int4v raw_buffer_load_b128(int4v rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.load.v4i32");

// Raw buffer resource over [p, p + bytes): loads past the end return zeros.
// Dword 3 = 0x00020000 is the gfx9-family raw-buffer format word.
struct BufRes {
  int lo, hi, bytes;
};
__device__ __forceinline__ BufRes make_res(const void* p, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return BufRes{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), (int)bytes};
}
// 16-byte buffer load; the descriptor is rebuilt from scalars at the use so the
// compiler keeps it in SGPRs (a descriptor it cannot prove uniform costs a
// waterfall loop per load and breaks its wait-count tracking).
__device__ __forceinline__ uint4 buf_load16(BufRes r, int voffset, int soffset) {
  int4v d;
  d.x = __builtin_amdgcn_readfirstlane(r.lo);
  d.y = __builtin_amdgcn_readfirstlane(r.hi);
  d.z = __builtin_amdgcn_readfirstlane(r.bytes);
  d.w = 0x00020000;
  return __builtin_bit_cast(uint4, raw_buffer_load_b128(d, voffset, __builtin_amdgcn_readfirstlane(soffset), 0));
}

typedef __attribute__((address_space(3))) void lds_void;
__device__ void raw_buffer_load_lds(int4v rsrc, lds_void* lds, int size, int voffset, int soffset, int offset,
                                    int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

// 16-byte buffer load straight into LDS (gfx950 buffer_load_dwordx4 ... lds): the
// wave's 64 lanes fill the 1 KB at lds_byte (a wave-uniform LDS byte address),
// lane j's 16 bytes at lds_byte + 16 j (established on the device). No VGPRs
// hold the data; the caller waits with wait_vmem() before the barrier that
// publishes the LDS region.
__device__ __forceinline__ void buf_load16_lds(BufRes r, uint32_t lds_byte, int voffset, int soffset) {
  int4v d;
  d.x = __builtin_amdgcn_readfirstlane(r.lo);
  d.y = __builtin_amdgcn_readfirstlane(r.hi);
  d.z = __builtin_amdgcn_readfirstlane(r.bytes);
  d.w = 0x00020000;
  raw_buffer_load_lds(d, (lds_void*)(uintptr_t)__builtin_amdgcn_readfirstlane(lds_byte), 16, voffset,
                      __builtin_amdgcn_readfirstlane(soffset), 0, 0);
}
// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left at their maxima): at most N vector
// memory loads still outstanding (loads complete in issue order)
template <int N = 0>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N <= 15, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}
// s_waitcnt vmcnt(N) for N up to 63 (gfx9 encoding: vmcnt bits [3:0] and [15:14]),
// expcnt and lgkmcnt left at their maxima
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(N >= 0 && N <= 63, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
// Workgroup barrier without the memory fence of __syncthreads (which waits for
// every outstanding load, direct-to-LDS loads in flight included). The caller
// waits for whatever the other waves must see (s_waitcnt) before it; the empty
// asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_no_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// LDS byte address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// Values of lanes l and l ^ 32 combined, through v_permlane32_swap (gfx950: a
// VALU exchange of the wave's two 32-lane halves, no LDS round trip). Both
// results of the swap hold one of the two lanes' values, so a symmetric op
// (max, sum) needs no knowledge of which is which.
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- attention dropout --------------------------------------------------------

// Keep decisions for attention dropout from a counter-based hash, so the forward
// and the backward regenerate the same mask without storing it. MurmurHash3's
// 32-bit finalizer (fmix32; A. Appleby, public domain) mixes
//   row(bh, q) = fmix32((bh * Sq + q) ^ seed_lo)                 (once per row)
//   u(q, k)    = fmix32(row + (k >> 1) * 0x9E3779B9 + seed_hi)   (one per key pair)
// and key k keeps iff its 16-bit half of u (low half for even k) is >= thr16,
// thr16 = round(p * 65536): P(keep) = 1 - thr16 / 65536. Kept weights are scaled
// by 1 / (1 - p). The host oracle restates these steps.
__device__ __forceinline__ uint32_t fmix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return h;
}
__device__ __forceinline__ uint32_t drop_row(uint32_t bh_sq_q, uint32_t seed_lo) { return fmix32(bh_sq_q ^ seed_lo); }
__device__ __forceinline__ uint32_t drop_pair(uint32_t row, int k, uint32_t seed_hi) {
  return fmix32(row + (uint32_t)(k >> 1) * 0x9E3779B9u + seed_hi);
}
__device__ __forceinline__ bool drop_keep(uint32_t u, int k, uint32_t thr16) {
  return ((k & 1) ? (u >> 16) : (u & 0xFFFFu)) >= thr16;
}

// ---- LDS tiles ---------------------------------------------------------------

// Byte offset of 16-byte chunk `chunk` of row `row` in a row-major DP-wide fp16 LDS
// tile, the chunk index XOR-swizzled by row. Two read patterns must be bank-
// conflict free (a pass of a wave's LDS read covers 256 bytes = all 64 banks):
//  (a) ds_read_b128 fragments: 16 lanes read one logical chunk of 16 consecutive
//      rows (16-aligned);
//  (b) ds_read_b64_tr_b16 fragments (tr_frag): 32 lanes read 4 consecutive chunks
//      (4-aligned) of 4 consecutive rows (4-aligned).
// 256-byte rows (every row starts at bank 0): chunk ^ g(row) with g the row's low
// 4 bits with their 2-bit halves swapped, a bijection on 16 rows for (a), and
// for (b) the 4 rows differ in g's top two bits, which move the 4-chunk group.
// 128-byte rows (row parity picks the bank half): chunk ^ h(row) with h a
// bijection on rows 2 apart for (a), whose top bit is row bit 1 for (b).
template <int DP>
__device__ __forceinline__ int swz_row(int row, int chunk) {
  if constexpr (DP >= 128) return row * (DP * 2) + ((chunk ^ (((row & 3) << 2) | ((row >> 2) & 3))) << 4);
  else return row * (DP * 2) + ((chunk ^ ((((row >> 1) & 1) << 2) | ((row >> 2) & 3))) << 4);
}

// Byte offset of the 8-byte run starting at column col (a multiple of 4).
template <int DP>
__device__ __forceinline__ int swz_run8(int row, int col) {
  return swz_row<DP>(row, col >> 3) + ((col >> 2) & 1) * 8;
}

// MFMA operand fragment (32 columns n x 16 k, either operand of
// v_mfma_f32_32x32x16_f16) of the TRANSPOSE of a row-major swizzled tile, read
// with two ds_read_b64_tr_b16 (gfx950): for lane L (n = L % 32, k group g = L / 32)
// k slot t holds tile[r0 + 4 g + (t & 3) + 8 (t >> 2)][c0 + n]. That k order is the
// one of a fragment packed from accumulators (rows 8 (t / 4) + 4 g + t % 4 of a
// 16-row step), so P or dS can be the other operand straight from registers.
// Within each 16-lane group the instruction gives element j of lane 4 a + b the
// b-th half of the 8 bytes addressed by lane a + 4 j; hence lane L addresses row
// r0 + 4 g + ((L / 4) % 4) (+ 8 for the second read), columns
// c0 + 16 ((L / 16) % 2) + 4 (L % 4).
template <int DP>
__device__ __forceinline__ half8 tr_frag(const uint8_t* tile, int r0, int c0, int lane) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  const int row = r0 + 4 * (lane >> 5) + ((lane >> 2) & 3);
  const int col = c0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(tile + swz_run8<DP>(row, col)));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(tile + swz_run8<DP>(row + 8, col)));
  return __builtin_bit_cast(half8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void stg16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

}  // namespace tbf16
