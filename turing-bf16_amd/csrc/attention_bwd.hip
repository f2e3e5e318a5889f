// Scaled attention backward on CDNA4 fp16 MFMA (flash-style, deterministic).
//
// Scaling (tbf16/autograd.py:166-193): e = max_{b,h}(frexp(amax dO[b,h]) + ev_q[b,h]),
// G = t_do - e, dO16 = fp16(dO * 2^(ev_q + G)); with q16 = q 2^a, k16 = k 2^-a,
// v16 = v 2^-ev (the workspace holds all four as zero-padded fp16 copies, rows to
// a multiple of 128 and columns to DP, written by one conversion pass and by the
// delta kernel, so the MFMA kernels stage plain fp16 with no conversion work):
//   P = exp2(S * scale * log2e - lse), dP = dO16 V16^T, delta = rowsum(dO16 * O16),
//   dS = P (dP - delta),
//   dv = bf16(sum_q P^T dO16 * 2^(-ev-G)), dk = bf16(scale * sum_q dS^T Q16 * 2^(-a-G)),
//   dq = bf16(scale * sum_k dS K16 * 2^(a-G)), each from fp32 accumulators.
// The fp16 values the reference's kernel would round its gradients to are
// scale * dS K16 (dq16), scale * dS^T Q16 (dk16) and P^T dO16 (dv16): the largest of
// their magnitudes goes to the `overflow` word (float bits, +inf if any is not
// finite); at 65520 and above the reference retries with t_do - 8
// (tbf16/autograd.py:184-187). A launch given a `gate` (the word of an earlier
// attempt at the same t_do) runs only if that attempt overflowed, at t_do - 8 r with
// r the retries the reference would take: all values scale by exactly 2^-8 per
// retry, so r follows from the earlier maximum. A gated launch skips prep (q16,
// k16, v16 and e are already in the workspace and exps_out) and its other kernels
// return at once when r = 0 (its overflow word then repeats the gate's), so the
// retry needs no host round trip.
//
// Kernels (4 waves, v_mfma_f32_32x32x16_f16):
//   prep:    q16, k16, v16 (one launch, memory-bound); its first block derives e, G.
//   delta:   one 16-lane group per query row; also writes dO16.
//   dkdv:    block = 128 keys of one query head's dK / dV (32 keys per wave, K16
//            fragments in registers, V16 rows in per-wave LDS), loops over
//            32-query tiles. Q and dO tiles sit in LDS row-major: the A operand
//            of S = Q K^T and dP = dO V^T (accumulators: each lane ONE key, 16
//            queries), and via ds_read_b64_tr_b16 the transposed B operand of
//            dV += P^T dO and dK += dS^T Q, so P / dS feed the MFMAs straight
//            from registers.
//   dq:      block = 128 queries (32 per wave, Q16 in registers, dO16 in per-wave
//            LDS), loops over 64-key tiles: K and V row-major in LDS; S^T and dP^T
//            give each lane ONE query, and dQ^T += K^T dS^T takes K^T fragments
//            from ds_read_b64_tr_b16.
//   kv_reduce (GQA only): with H > Hkv, dkdv writes each query head's dK / dV in
//            fp32 and this pass sums a group's heads in head order and rounds once
//            to bf16 (the reference's fp32 _reduce_kv, tbf16/autograd.py:141-146),
//            so the overflow check sees every query head's dk16 / dv16 before the
//            sum, as the reference checks its per-head fp16 gradients.
#include <algorithm>
#include <math.h>

#include "abi_util.h"
#include "common.h"

using namespace tbf16;

namespace tbf16 {
int64_t head_amax_chunks(int64_t BH, int64_t S);
int launch_head_amax_partial(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                             int64_t sh, int64_t ss, float* partial, int64_t nchunks, hipStream_t st);
}  // namespace tbf16

namespace {

constexpr int NTH = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kF16Overflow = 65520.f;

struct BwdParams {
  const uint16_t *q, *k, *v, *o16, *dout;
  const float* lse;
  const int32_t* exps_fwd;  // {a, 0, ev[b*Hkv + hk]...}
  int64_t q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, d_sb, d_sh, d_ss;
  const uint16_t* bias;
  int64_t bias_sb, bias_sh, bias_sq;
  int B, H, Hkv, Sq, Sk, D;
  float scale, scale_log2;
  int causal;
  int t_do;
  const float* part_do;
  int nch_do;
  float* delta;     // (B, H, Sq)
  // zero-padded fp16 copies: (B, H, Sqp, DP) for q16 / do16, (B, Hkv, Skp, DP) for k16 / v16
  uint16_t *q16, *k16, *v16, *do16;
  int Sqp, Skp, DPc;
  int32_t* exps_out;  // {e, G}
  int32_t* overflow;      // largest fp16 intermediate magnitude (float bits), this attempt
  const int32_t* gate;    // null, or an earlier attempt's `overflow` word (see above)
  uint16_t *dq, *dk, *dv;
  // GQA (H > Hkv): per-query-head fp32 dK / dV (B, H, Sk, D), summed by kv_reduce
  float *dk_part, *dv_part;
  // dropout of the forward pass (DROP kernels regenerate its keep mask)
  uint32_t drop_lo, drop_hi, drop_thr;
  float drop_scale;
};


__device__ __forceinline__ int ev_of(const BwdParams& p, int b, int h) {
  return p.exps_fwd[2 + b * p.Hkv + h / (p.H / p.Hkv)];
}

// e = max over (b, h) of frexp(amax dO[b,h]) + ev_q[b,h]  (block-wide)
// (wave-parallel: wave w reduces heads w, w + 4, ..., a lane per chunk, eight
// heads' loads in flight before any is reduced)
__device__ int compute_e(const BwdParams& p, int* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nbh = p.B * p.H, nch = p.nch_do;
  int e = INT_MIN;
  for (int bh0 = wave; bh0 < nbh; bh0 += 32) {
    float m[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = 0.f;
    for (int c = lane; c < nch; c += 64) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int bh = bh0 + 4 * j;
        if (bh < nbh) m[j] = fmaxf(m[j], p.part_do[bh * nch + c]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int bh = bh0 + 4 * j;
      const float mx = wave_max(m[j]);
      if (bh < nbh) e = max(e, frexp_exp(mx) + ev_of(p, bh / p.H, bh % p.H));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) e = max(e, __shfl_xor(e, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = e;
  __syncthreads();
  return max(max(red[0], red[1]), max(red[2], red[3]));
}

// Retries the reference takes after an attempt whose largest fp16 intermediate had
// magnitude x (the bits of a non-negative float, +inf / NaN when not finite): the
// first r with x 2^(-8 r) < 65520, at most kAttnRetries - 1.
constexpr int kAttnRetries = 6;
__device__ __forceinline__ int retries_after(int32_t bits) {
  float x = __int_as_float(bits);
  int r = 0;
  while (r < kAttnRetries - 1 && !(x < kF16Overflow)) {
    x *= 0x1p-8f;
    ++r;
  }
  return r;
}
// a gated launch whose gate needs no retry does nothing
__device__ __forceinline__ bool gated_off(const BwdParams& p) { return p.gate && retries_after(*p.gate) == 0; }
// Largest |x| seen by the wave (non-finite as +inf) into the attempt's overflow word:
// float bits of non-negative values order as integers.
__device__ __forceinline__ void record_max(const BwdParams& p, float mx, bool nonfinite) {
  int bits = nonfinite ? 0x7f800000 : __float_as_int(mx);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) bits = max(bits, __shfl_xor(bits, o, 64));
  if ((threadIdx.x & 63) == 0 && bits > 0) atomicMax(p.overflow, bits);
}

// ---- q16 = fp16(q 2^a), k16 = fp16(k 2^-a), v16 = fp16(v 2^-ev), and {e, G} -----
// Grid: x = groups of 4 x 256 / (DP / 8) padded rows, y = (copy, batch, head) with the
// q heads first, then the k and v heads. Zeros past the real rows and columns.
// Block (0, 0) also derives e and G (they are needed by the delta pass only).
__global__ __launch_bounds__(NTH) void prep_kernel(BwdParams p) {
  __shared__ int red[4];
  if (blockIdx.x == 0 && blockIdx.y == 0) {
    const int e = compute_e(p, red);
    if (threadIdx.x == 0) {
      p.exps_out[0] = e;
      p.exps_out[1] = p.t_do - e;
      *p.overflow = 0;  // the MFMA kernels of this attempt raise it
    }
  }
  const int CPR = p.DPc / 8;
  const int nq = p.B * p.H, nk = p.B * p.Hkv;
  const int y = blockIdx.y;
  const int seg = y < nq ? 0 : y < nq + nk ? 1 : 2;
  const int bh = seg == 0 ? y : seg == 1 ? y - nq : y - nq - nk;
  const int HH = seg == 0 ? p.H : p.Hkv, b = bh / HH, h = bh % HH;
  const int Sp = seg == 0 ? p.Sqp : p.Skp, S = seg == 0 ? p.Sq : p.Sk;
  const int a = p.exps_fwd[0];
  const int e = seg == 0 ? a : seg == 1 ? -a : -p.exps_fwd[2 + bh];
  const float sc = ldexp1(e);
  const uint16_t* src = seg == 0   ? p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh
                        : seg == 1 ? p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh
                                   : p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  const int64_t ss = seg == 0 ? p.q_ss : seg == 1 ? p.k_ss : p.v_ss;
  uint16_t* dst = (seg == 0 ? p.q16 : seg == 1 ? p.k16 : p.v16) + (int64_t)bh * Sp * p.DPc;
  // four rows per thread, all loads issued before the stores
  const int rpb = NTH / CPR, ch = threadIdx.x % CPR;
  const int row0 = blockIdx.x * 4 * rpb + threadIdx.x / CPR;
  uint4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = row0 + i * rpb;
    v[i] = row < S && ch * 8 < p.D ? ldg16(src + (int64_t)row * ss + ch * 8) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = row0 + i * rpb;
    if (row < Sp) stg16(dst + (int64_t)row * p.DPc + ch * 8, cvt_bf16x8_f16x8(v[i], sc));
  }
}

// ---- delta = rowsum(dO16 * O16), and dO16 ------------------------------------------
// One 16-lane group per padded query row; G comes from the prep pass.
__global__ __launch_bounds__(NTH) void delta_kernel(BwdParams p) {
  if (gated_off(p)) {
    // nothing to redo: the outputs are the earlier attempt's, and so is this
    // call's overflow word (below 65520)
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *p.overflow = *p.gate;
    return;
  }
  // a gated retry (no prep launch): G at the retried t_do from the first attempt's
  // e; block (0, 0) publishes it for the MFMA kernels and clears the overflow word
  int G;
  if (p.gate) {
    G = p.t_do - 8 * retries_after(*p.gate) - p.exps_out[0];
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
      p.exps_out[1] = G;
      *p.overflow = 0;
    }
  } else {
    G = p.exps_out[1];
  }
  const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
  const float sdo = ldexp1(ev_of(p, b, h) + G);
  const int row = blockIdx.x * 16 + (threadIdx.x >> 4), l16 = threadIdx.x & 15;
  float acc = 0.f;
  // dO16 row (zeros past Sq and past D), 8 columns per lane
  uint16_t* wrow = p.do16 + ((int64_t)bh * p.Sqp + row) * p.DPc;
  for (int c = l16 * 8; c < p.DPc; c += 128)
    if (row < p.Sqp && (row >= p.Sq || c >= p.D)) stg16(wrow + c, make_uint4(0, 0, 0, 0));
  if (row < p.Sq) {
    const uint16_t* dr = p.dout + (int64_t)b * p.d_sb + (int64_t)h * p.d_sh + (int64_t)row * p.d_ss;
    const uint16_t* orow = p.o16 + ((int64_t)bh * p.Sq + row) * p.D;
    for (int d = l16 * 8; d < p.D; d += 128) {
      const uint4 dv = cvt_bf16x8_f16x8(ldg16(dr + d), sdo);
      stg16(wrow + d, dv);
      const uint4 ov = ldg16(orow + d);
      acc += f16_lo(dv.x) * f16_lo(ov.x) + f16_hi(dv.x) * f16_hi(ov.x) + f16_lo(dv.y) * f16_lo(ov.y) +
             f16_hi(dv.y) * f16_hi(ov.y) + f16_lo(dv.z) * f16_lo(ov.z) + f16_hi(dv.z) * f16_hi(ov.z) +
             f16_lo(dv.w) * f16_lo(ov.w) + f16_hi(dv.w) * f16_hi(ov.w);
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (row < p.Sq && l16 == 0) p.delta[(int64_t)bh * p.Sq + row] = acc;
}

// ---- dK, dV --------------------------------------------------------------------
// Block = 128 keys of one query head (32 per wave, K16 fragments in registers, the
// wave's V16 rows in a private LDS region), loop over 32-query tiles,
// double-buffered in LDS by direct global -> LDS loads. Q16 and
// dO16 tiles sit in LDS once, row-major: they are the A operand of S = Q K^T and
// dP = dO V^T (lane = ONE key, 16 queries), and their transposes for dV += P^T dO
// and dK += dS^T Q come from ds_read_b64_tr_b16, so P and dS feed the MFMAs
// straight from registers. Without a bias or dropout (and at DP <= 128) a wave
// stays within 256 registers and two blocks share a CU.
// PART 0 accumulates dK and dV together; for DP = 256 (whose two accumulator
// sets and K fragments exceed a wave's 512 registers) PART 1 accumulates dV and
// PART 2 dK, in two launches that each recompute S.
// DROP: the forward's dropout mask regenerated from (seed, row, key): dV takes
// P o Z and dS = P o (Z o dP - delta), Z = keep / (1 - p).
// GQA: the block's query head h reads kv head h / (H / Hkv) and writes its scaled
// fp32 dK / dV to dk_part / dv_part; kv_reduce sums the group. The block's overflow
// maximum is then one query head's, as the reference checks dk16 / dv16 per head.
template <int DP, bool CAUSAL, bool HAS_BIAS, int PART, bool DROP>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(HAS_BIAS || DROP || DP > 128 ? 1 : 2,
                                                                     HAS_BIAS || DROP || DP > 128 ? 1 : 2))) void
dkdv_kernel(BwdParams p) {
  if (gated_off(p)) return;
  constexpr bool WANT_DV = PART != 2, WANT_DK = PART != 1;
  constexpr int BQ = 32, BK = 128;
  constexpr int KS = DP / 16, DB = DP / 32, CPR = DP / 8;
  constexpr int TILE = BQ * DP * 2;   // one 32 x DP fp16 tile
  constexpr int VW = 32 * DP * 2;     // one wave's V rows
  constexpr int STG = 2 * TILE;       // one stage: Q16 and dO16 tiles
  // stages filled by direct global -> LDS loads, 1 KB per wave instruction
  constexpr int NBLK = STG / 1024, QBLK = TILE / 1024, BPW = NBLK / (NTH / 64);
  static_assert(NBLK % (NTH / 64) == 0 && QBLK % BPW == 0, "stage blocks");
  // V rows of the four waves (also the epilogue's staging, 64 keys per pass), and
  // the two stages as separate objects: the compiler's LDS alias analysis then
  // sees that reads of one stage never wait for the loads into the other
  __shared__ __align__(1024) uint8_t smem[4 * VW];
  __shared__ __align__(1024) uint8_t sst0[STG];
  __shared__ __align__(1024) uint8_t sst1[STG];
  __shared__ __align__(16) float s_lse[2][BQ];
  __shared__ __align__(16) float s_delta[2][BQ];
  __shared__ __align__(16) uint32_t s_drow[DROP ? 2 : 1][BQ];  // dropout row hashes

  const int tid = threadIdx.x, lane = tid & 63, fr = lane & 31, fk = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // grid (query heads, key blocks): dispatch runs over heads first, so every
  // head's heaviest key blocks (the most query tiles under a causal mask) go out first
  const int bh = blockIdx.x, b = bh / p.H, h = bh % p.H;
  const int bk = b * p.Hkv + h / (p.H / p.Hkv);  // the kv head
  const int k0 = blockIdx.y * BK;
  const int a = p.exps_fwd[0];
  const int ev = p.exps_fwd[2 + bk];
  const int G = p.exps_out[1];

  // wave's 32 keys: K16 fragments (B operand of S = Q K^T) in registers, V16 rows
  // (B operand of dP = dO V^T) in this wave's LDS region
  const int key = k0 + wave * 32 + fr;
  half8 kf[KS];
  uint8_t* sVw = smem + wave * VW;
  {
    // padded copies: key < Skp and d < DP always lie inside
    const uint16_t* kr = p.k16 + ((int64_t)bk * p.Skp + key) * DP;
    const uint16_t* vr = p.v16 + ((int64_t)bk * p.Skp + key) * DP;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d = 16 * s + 8 * fk;
      kf[s] = __builtin_bit_cast(half8, ldg16(kr + d));
      *reinterpret_cast<uint4*>(sVw + swz_row<DP>(fr, 2 * s + fk)) = ldg16(vr + d);
    }
  }
  floatx16 dk[WANT_DK ? DB : 1], dv[WANT_DV ? DB : 1];
#pragma unroll
  for (int i = 0; i < (WANT_DK ? DB : 1); ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[i][r] = 0.f;
#pragma unroll
  for (int i = 0; i < (WANT_DV ? DB : 1); ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[i][r] = 0.f;

  const int nqt = (p.Sq + BQ - 1) / BQ;
  const int qt0 = CAUSAL ? min(k0 / BQ, nqt) : 0;
  const int total = nqt - qt0;

  // Query tiles of 32 rows in two LDS stages (tile it in stage it % 2). When tile
  // it starts, threads < 32 load tile it + 1's lse and delta into registers (for
  // s_lse / s_delta after tile it's S / dP products) and then every wave issues
  // its share of tile it + 1's Q16 and dO16 rows as direct global -> LDS loads
  // (lane j of an instruction lands at byte 16 j of its 1 KB block, so the row
  // swizzle is applied on the source side); the barrier that ends tile it waits
  // for them.
  int voff[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int byte = ((wave * BPW + i) % QBLK) * 1024 + 16 * lane, row = byte / (2 * DP), phys = (byte % (2 * DP)) >> 4;
    const int lch = (swz_row<DP>(row, phys) - row * 2 * DP) >> 4;  // the XOR swizzle is its own inverse
    voff[i] = (row * DP + lch * 8) * 2;
  }
  float rl = INFINITY, rdl = 0.f;
  uint32_t rdr = 0u;
  auto gload = [&](int it, uint8_t* stage) {
    const int q0 = (qt0 + it) * BQ;
    if (tid < BQ) {
      const int qi = q0 + tid;
      rl = qi < p.Sq ? p.lse[(int64_t)bh * p.Sq + qi] : INFINITY;
      rdl = qi < p.Sq ? p.delta[(int64_t)bh * p.Sq + qi] : 0.f;
      if constexpr (DROP) rdr = drop_row((uint32_t)bh * (uint32_t)p.Sq + (uint32_t)qi, p.drop_lo);
    }
    const int64_t row0 = ((int64_t)bh * p.Sqp + q0) * DP;
    // blocks [0, QBLK) of a stage hold Q16 rows, the rest dO16 rows; a wave's
    // BPW blocks all lie on one side (QBLK is a multiple of BPW)
    const BufRes res = make_res((wave * BPW < QBLK ? p.q16 : p.do16) + row0, TILE);
    const uint32_t base = lds_addr(stage);
#pragma unroll
    for (int i = 0; i < BPW; ++i) buf_load16_lds(res, base + (wave * BPW + i) * 1024, voff[i], 0);
  };
  auto lstore = [&](int stg) {
    if (tid < BQ) {
      s_lse[stg][tid] = rl;
      s_delta[stg][tid] = rdl;
      if constexpr (DROP) s_drow[stg][tid] = rdr;
    }
  };

  if (total > 0) {
    gload(0, sst0);
    lstore(0);
  }
  wait_vmem();
  __syncthreads();
  auto tile = [&](int it, const uint8_t* sQ, uint8_t* snext, int stg) {
    const int q0 = (qt0 + it) * BQ;
    const uint8_t* sD = sQ + TILE;
    const bool more = it + 1 < total;
    if (more) gload(it + 1, snext);

    const bool edge = q0 + BQ > p.Sq || k0 + BK > p.Sk || (CAUSAL && k0 + wave * 32 + 31 >= q0);
    // with a bias the logits are scaled and biased first, as in the forward pass
    const float cs = HAS_BIAS ? 1.f : p.scale_log2;
    // S and dP for the tile's 32 queries: lane = one key, 16 queries
    floatx16 sacc, pacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const half8 qa = *reinterpret_cast<const half8*>(sQ + swz_row<DP>(fr, 2 * s + fk));
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa, kf[s], sacc, 0, 0, 0);
      if constexpr (WANT_DK) {  // dP is needed only for dS
        const half8 da = *reinterpret_cast<const half8*>(sD + swz_row<DP>(fr, 2 * s + fk));
        const half8 vb = *reinterpret_cast<const half8*>(sVw + swz_row<DP>(fr, 2 * s + fk));
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(da, vb, pacc, 0, 0, 0);
      }
    }
    // fragment reads one k step ahead of the MFMAs that use them
    constexpr int RPS = WANT_DK ? 3 : 1, MPS = WANT_DK ? 2 : 1;  // reads, MFMAs per k step
    __builtin_amdgcn_sched_group_barrier(0x100, RPS, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      __builtin_amdgcn_sched_group_barrier(0x008, MPS, 0);
      if (s + 1 < KS) __builtin_amdgcn_sched_group_barrier(0x100, RPS, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the next tile's lse and delta: their slots' reads retired at the previous barrier
    if (more) lstore(stg ^ 1);
    if constexpr (HAS_BIAS) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = q0 + 8 * (r >> 2) + 4 * fk + (r & 3);
        if (qi < p.Sq && key < p.Sk)
          sacc[r] = sacc[r] * p.scale_log2 +
                    (float)__builtin_bit_cast(_Float16, p.bias[(int64_t)b * p.bias_sb + (int64_t)h * p.bias_sh +
                                                               (int64_t)qi * p.bias_sq + key]) * kLog2e;
        else
          sacc[r] *= p.scale_log2;
      }
    }
    // masking only where the tile crosses the diagonal or an end
    if (edge) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = q0 + 8 * (r >> 2) + 4 * fk + (r & 3);
        if (key >= p.Sk || qi >= p.Sq || (CAUSAL && key > qi)) sacc[r] = -INFINITY;
      }
    }
    // P and dS (fp16, packed in MFMA k-slot order); the lane's 16 queries are 4
    // runs of 4 (q = 8 i + 4 fk + j), so lse and delta come as float4s
    uint32_t pp[8], ds[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ql0 = 8 * i + 4 * fk;
      const float4 l4 = *reinterpret_cast<const float4*>(&s_lse[stg][ql0]);
      const float4 d4 = *reinterpret_cast<const float4*>(&s_delta[stg][ql0]);
      const float lse4[4] = {l4.x, l4.y, l4.z, l4.w}, del4[4] = {d4.x, d4.y, d4.z, d4.w};
      float pv[4], dsv[4], pz[4];
      uint4 dr4 = make_uint4(0, 0, 0, 0);
      if constexpr (DROP) dr4 = *reinterpret_cast<const uint4*>(&s_drow[DROP ? stg : 0][ql0]);
      const uint32_t dr[4] = {dr4.x, dr4.y, dr4.z, dr4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[j] = __builtin_amdgcn_exp2f(fmaf(sacc[4 * i + j], cs, -lse4[j]));
        float dpj = WANT_DK ? pacc[4 * i + j] : 0.f;
        pz[j] = pv[j];
        if constexpr (DROP) {
          const bool keep = drop_keep(drop_pair(dr[j], key, p.drop_hi), key, p.drop_thr);
          pz[j] = keep ? pv[j] : 0.f;  // 1 / (1 - p) is applied to dV in fp32 at the end
          dpj = keep ? dpj * p.drop_scale : 0.f;
        }
        dsv[j] = WANT_DK ? pv[j] * (dpj - del4[j]) : 0.f;
      }
      pp[2 * i] = pack_f16(pz[0], pz[1]);
      pp[2 * i + 1] = pack_f16(pz[2], pz[3]);
      ds[2 * i] = pack_f16(dsv[0], dsv[1]);
      ds[2 * i + 1] = pack_f16(dsv[2], dsv[3]);
    }
    // dV += P^T dO16, dK += dS^T Q16 over the tile's two 16-query steps
#pragma unroll
    for (int kq = 0; kq < 2; ++kq) {
      const int o = 4 * kq, r0 = 16 * kq;
      const half8 pa = __builtin_bit_cast(half8, make_uint4(pp[o], pp[o + 1], pp[o + 2], pp[o + 3]));
      const half8 sa = __builtin_bit_cast(half8, make_uint4(ds[o], ds[o + 1], ds[o + 2], ds[o + 3]));
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        if constexpr (WANT_DV) {
          const half8 dob = tr_frag<DP>(sD, r0, db * 32, lane);
          dv[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, dob, dv[db], 0, 0, 0);
        }
        if constexpr (WANT_DK) {
          const half8 qbf = tr_frag<DP>(sQ, r0, db * 32, lane);
          dk[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa, qbf, dk[db], 0, 0, 0);
        }
      }
    }
    // transposed reads one (kq, db) step ahead of their MFMAs
    constexpr int TRS = PART == 0 ? 4 : 2, TMS = PART == 0 ? 2 : 1;
    __builtin_amdgcn_sched_group_barrier(0x100, TRS, 0);
#pragma unroll
    for (int s = 0; s + 1 < 2 * DB; ++s) {
      __builtin_amdgcn_sched_group_barrier(0x100, TRS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, TMS, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, TMS, 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();
    __syncthreads();
  };
  for (int it = 0; it < total; it += 2) {
    tile(it, sst0, sst1, 0);
    if (it + 1 < total) tile(it + 1, sst1, sst0, 1);
  }

  // ---- epilogue: lane = key row (fr), d = db*32 + 8*(r/4) + 4*fk + r%4 ----
  // dV / dK accumulators are C[key][d] with key = MFMA row: lane holds col d = fr and
  // rows key = 8*(r/4) + 4*fk + r%4. Transpose through LDS for 16-byte stores, 64
  // keys (two waves' rows) per pass.
  __syncthreads();
  float* sOut = reinterpret_cast<float*>(smem);  // 64 keys x DP floats
  const float sk_out = ldexp1(-a - G) * p.scale, sv_out = ldexp1(-ev - G);
  float mx = 0.f;  // largest |dk16| / |dv16| of this thread
  bool nonfinite = false;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int kind = pass >> 1, half = pass & 1;
    if ((kind == 0 && !WANT_DV) || (kind == 1 && !WANT_DK)) continue;
    floatx16* acc = kind == 0 ? dv : dk;
    // dV accumulated P o keep: the dropout scale 1 / (1 - p) comes in here, in fp32
    const float dzs = DROP ? p.drop_scale : 1.f;
    const float so = kind == 0 ? sv_out * dzs : sk_out;
    const float chk = kind == 0 ? dzs : p.scale;
    if ((wave >> 1) == half) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kl = (wave & 1) * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
          const int d = db * 32 + fr;
          const float x = acc[db][r];
          if (k0 + half * 64 + kl < p.Sk && d < p.D) {
            const float ax = fabsf(x * chk);
            mx = fmaxf(mx, ax);
            nonfinite |= !(ax <= __FLT_MAX__);
          }
          sOut[kl * DP + d] = x * so;
        }
    }
    __syncthreads();
    uint16_t* out = kind == 0 ? p.dv : p.dk;
    float* part = kind == 0 ? p.dv_part : p.dk_part;  // GQA: this query head's fp32 share
    for (int i = tid; i < 64 * (DP / 8); i += NTH) {
      const int kl = i / (DP / 8), d = (i % (DP / 8)) * 8;
      const int kk = k0 + half * 64 + kl;
      if (kk < p.Sk && d < p.D) {
        const float* src = sOut + kl * DP + d;
        if (part) {
          float* dst = part + ((int64_t)bh * p.Sk + kk) * p.D + d;
          *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(src);
          *reinterpret_cast<float4*>(dst + 4) = *reinterpret_cast<const float4*>(src + 4);
        } else {
          stg16(out + ((int64_t)bk * p.Sk + kk) * p.D + d,
                make_uint4(pack_bf16(src[0], src[1]), pack_bf16(src[2], src[3]), pack_bf16(src[4], src[5]),
                           pack_bf16(src[6], src[7])));
        }
      }
    }
    __syncthreads();
  }
  record_max(p, mx, nonfinite);
}

// ---- GQA: dK / dV = sum over a group's query heads -------------------------------
// part: (B, H, Sk, D) fp32, already scaled; out: (B, Hkv, Sk, D) bf16. One thread per
// 8 elements, the heads added in order g = 0 .. group - 1, one bf16 rounding.
__global__ __launch_bounds__(NTH) void kv_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ out,
                                                        int group, int64_t per_head, int64_t n8, const int32_t* gate) {
  if (gate && retries_after(*gate) == 0) return;  // a gated launch with nothing to redo
  const int64_t i = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (i >= n8) return;
  const int64_t e = i * 8, bk = e / per_head, r = e % per_head;
  const float* src = part + bk * group * per_head + r;
  float4 lo = *reinterpret_cast<const float4*>(src), hi = *reinterpret_cast<const float4*>(src + 4);
  for (int g = 1; g < group; ++g) {
    const float4 l = *reinterpret_cast<const float4*>(src + g * per_head);
    const float4 h = *reinterpret_cast<const float4*>(src + g * per_head + 4);
    lo.x += l.x; lo.y += l.y; lo.z += l.z; lo.w += l.w;
    hi.x += h.x; hi.y += h.y; hi.z += h.z; hi.w += h.w;
  }
  stg16(out + e, make_uint4(pack_bf16(lo.x, lo.y), pack_bf16(lo.z, lo.w), pack_bf16(hi.x, hi.y),
                            pack_bf16(hi.z, hi.w)));
}

// ---- dQ --------------------------------------------------------------------------
// Two blocks per CU (two waves per SIMD, without a bias): a wave's dO rows live in
// a private LDS region instead of registers, and K/V arrive in 32-key tiles
// (double-buffered, direct global -> LDS loads), which keeps a wave within 256
// registers.
template <int DP, bool CAUSAL, bool HAS_BIAS, bool DROP>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(HAS_BIAS || DP > 128 ? 1 : 2, HAS_BIAS || DP > 128 ? 1 : 2))) void
dq_kernel(BwdParams p) {
  if (gated_off(p)) return;
  constexpr int BQ = 128, BKV = 32;
  constexpr int KS = DP / 16, DB = DP / 32;
  constexpr int TILE = BKV * DP * 2;  // 32 key rows of K16 (or V16)
  constexpr int STG = 2 * TILE;       // one stage: K16 rows, then V16 rows
  constexpr int NBLK = STG / 1024, KBLK = TILE / 1024, BPW = NBLK / (NTH / 64);
  static_assert(NBLK % (NTH / 64) == 0 && KBLK % BPW == 0, "stage blocks");
  constexpr int DOW = 32 * DP * 2;  // one wave's dO rows
  // per-wave dO rows and two K/V stages as separate objects (the compiler's LDS
  // alias analysis then sees that reads of one stage never wait for the direct
  // loads into the other)
  __shared__ __align__(1024) uint8_t smem[4 * DOW];
  __shared__ __align__(1024) uint8_t sst0[STG];
  __shared__ __align__(1024) uint8_t sst1[STG];

  const int tid = threadIdx.x, lane = tid & 63, fr = lane & 31, fk = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // grid (heads, query blocks), heaviest query blocks of every head first
  const int bh = blockIdx.x, b = bh / p.H, h = bh % p.H, hk = h / (p.H / p.Hkv);
  const int qt = CAUSAL ? (int)(gridDim.y - 1 - blockIdx.y) : (int)blockIdx.y;
  const int q0 = qt * BQ;
  const int a = p.exps_fwd[0];
  const int ev = p.exps_fwd[2 + b * p.Hkv + hk];
  const int G = p.exps_out[1];

  const int qrow = q0 + wave * 32 + fr;
  half8 qf[KS];
  uint8_t* sDo = smem + wave * DOW;  // written and read by this wave only
  {
    // padded copies: qrow < Sqp and d < DP always lie inside
    const uint16_t* qr = p.q16 + ((int64_t)bh * p.Sqp + qrow) * DP;
    const uint16_t* dr = p.do16 + ((int64_t)bh * p.Sqp + qrow) * DP;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d = 16 * s + 8 * fk;
      qf[s] = __builtin_bit_cast(half8, ldg16(qr + d));
      *reinterpret_cast<uint4*>(sDo + swz_row<DP>(fr, 2 * s + fk)) = ldg16(dr + d);
    }
  }
  const float lse_q = qrow < p.Sq ? p.lse[(int64_t)bh * p.Sq + qrow] : INFINITY;
  const float delta_q = qrow < p.Sq ? p.delta[(int64_t)bh * p.Sq + qrow] : 0.f;
  const uint32_t drow = DROP ? drop_row((uint32_t)bh * (uint32_t)p.Sq + (uint32_t)qrow, p.drop_lo) : 0u;
  floatx16 dq[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;

  // 32-key tiles in two stages (tile t in stage t % 2), the padded copies (zeros
  // past Sk and D) copied global -> LDS directly: lane j of a wave instruction
  // lands at byte 16 j of its 1 KB block, so the row swizzle is applied on the
  // source side. Tile t + 1's loads go out when tile t starts; the barrier that
  // ends tile t waits for them.
  const int nk = CAUSAL ? min(p.Sk, min(q0 + BQ, p.Sq)) : p.Sk;
  const int nt = (nk + BKV - 1) / BKV;
  int voff[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int byte = ((wave * BPW + i) % KBLK) * 1024 + 16 * lane, row = byte / (2 * DP), phys = (byte % (2 * DP)) >> 4;
    const int lch = (swz_row<DP>(row, phys) - row * 2 * DP) >> 4;  // the XOR swizzle is its own inverse
    voff[i] = (row * DP + lch * 8) * 2;
  }
  const uint16_t* kvsrc = (wave * BPW < KBLK ? p.k16 : p.v16) + (int64_t)(b * p.Hkv + hk) * p.Skp * DP;
  auto dload = [&](uint8_t* stage, int t) {
    const BufRes res = make_res(kvsrc + (int64_t)t * BKV * DP, TILE);
    const uint32_t base = lds_addr(stage);
#pragma unroll
    for (int i = 0; i < BPW; ++i) buf_load16_lds(res, base + (wave * BPW + i) * 1024, voff[i], 0);
  };
  const uint16_t* brow = nullptr;
  if constexpr (HAS_BIAS)
    brow = p.bias + (int64_t)b * p.bias_sb + (int64_t)h * p.bias_sh + (int64_t)min(qrow, p.Sq - 1) * p.bias_sq;

  // one 32-key tile: S^T and dP^T (lane = one query, 16 keys), then dS and its
  // two 16-key steps of dQ^T += K^T dS^T
  const float cs = HAS_BIAS ? 1.f : p.scale_log2;  // with a bias: scaled and biased first
  auto tile = [&](int t, const uint8_t* sK, uint8_t* snext) {
    if (t + 1 < nt) dload(snext, t + 1);
    const uint8_t* sV = sK + TILE;
    {
      floatx16 sacc, pacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const half8 ka = *reinterpret_cast<const half8*>(sK + swz_row<DP>(fr, 2 * s + fk));
        const half8 va = *reinterpret_cast<const half8*>(sV + swz_row<DP>(fr, 2 * s + fk));
        const half8 dfs = *reinterpret_cast<const half8*>(sDo + swz_row<DP>(fr, 2 * s + fk));
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[s], sacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, dfs, pacc, 0, 0, 0);
      }
      // fragment reads one k step ahead of the MFMAs that use them
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
      for (int s = 0; s + 1 < KS; ++s) {
        __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_barrier(0);
      const int kb0 = t * BKV;
      if constexpr (HAS_BIAS) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = kb0 + 8 * (r >> 2) + 4 * fk + (r & 3);
          sacc[r] = sacc[r] * p.scale_log2 + (kk < p.Sk ? (float)__builtin_bit_cast(_Float16, brow[kk]) * kLog2e : 0.f);
        }
      }
      // masking only where the tile crosses the diagonal or an end
      if (kb0 + BKV > p.Sk || q0 + BQ > p.Sq || (CAUSAL && kb0 + BKV - 1 > q0 + wave * 32)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = kb0 + 8 * (r >> 2) + 4 * fk + (r & 3);
          if (kk >= p.Sk || qrow >= p.Sq || (CAUSAL && kk > qrow)) sacc[r] = -INFINITY;
        }
      }
      uint32_t ds[8];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[r], cs, -lse_q));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[r + 1], cs, -lse_q));
        float dp0 = pacc[r], dp1 = pacc[r + 1];
        if constexpr (DROP) {  // dS = P o (Z o dP - delta)
          const int kk = kb0 + 8 * (r >> 2) + 4 * fk + (r & 3);  // even
          const uint32_t u = drop_pair(drow, kk, p.drop_hi);
          dp0 = drop_keep(u, kk, p.drop_thr) ? dp0 * p.drop_scale : 0.f;
          dp1 = drop_keep(u, kk + 1, p.drop_thr) ? dp1 * p.drop_scale : 0.f;
        }
        ds[r >> 1] = pack_f16(p0 * (dp0 - delta_q), p1 * (dp1 - delta_q));
      }
#pragma unroll
      for (int kq = 0; kq < 2; ++kq) {
        const int o = 4 * kq;
        const half8 sa = __builtin_bit_cast(half8, make_uint4(ds[o], ds[o + 1], ds[o + 2], ds[o + 3]));
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const half8 kbf = tr_frag<DP>(sK, 16 * kq, db * 32, lane);  // K^T fragment
          dq[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kbf, sa, dq[db], 0, 0, 0);
        }
      }
      // transposed reads one d block ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int s = 0; s + 1 < 2 * DB; ++s) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmem();
    __syncthreads();
  };
  if (nt > 0) dload(sst0, 0);
  wait_vmem();
  __syncthreads();
  for (int t = 0; t < nt; t += 2) {
    tile(t, sst0, sst1);
    if (t + 1 < nt) tile(t + 1, sst1, sst0);
  }

  // dQ^T accumulators: lane col = query (fr), rows d = db*32 + 8*(r/4) + 4*fk + r%4
  float mx = 0.f;  // largest |dq16| of this thread
  bool nonfinite = false;
  if (qrow < p.Sq) {
    const float so = ldexp1(a - G) * p.scale;
    const int64_t orow = ((int64_t)bh * p.Sq + qrow) * p.D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + 8 * rq + 4 * fk;
        if (d >= p.D) continue;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = dq[db][4 * rq + e];
          const float ax = fabsf(x * p.scale);
          mx = fmaxf(mx, ax);
          nonfinite |= !(ax <= __FLT_MAX__);
          y[e] = x * so;
        }
        *reinterpret_cast<uint2*>(p.dq + orow + d) = make_uint2(pack_bf16(y[0], y[1]), pack_bf16(y[2], y[3]));
      }
  }
  record_max(p, mx, nonfinite);
}

struct BwdWs {
  int64_t nch, Sqp, Skp, DP;
  size_t off_delta, off_q16, off_do16, off_k16, off_v16, off_dkp, off_dvp, total;
};

// partial dO maxima | delta (B, H, Sq) fp32 | q16, dO16 (B, H, Sqp, DP) | k16, v16
// (B, Hkv, Skp, DP), rows padded to a multiple of 128, DP = 64, 128 or 256 | with
// GQA only, the per-query-head fp32 dK and dV (B, H, Sk, D)
BwdWs bwd_ws(int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D) {
  BwdWs w;
  w.nch = head_amax_chunks(B * H, Sq);
  w.Sqp = cdiv(Sq, 128) * 128;
  w.Skp = cdiv(Sk, 128) * 128;
  w.DP = D <= 64 ? 64 : D <= 128 ? 128 : 256;
  w.off_delta = align_up((size_t)(B * H * w.nch) * 4, 256);
  w.off_q16 = w.off_delta + align_up((size_t)(B * H * Sq) * 4, 256);
  const size_t qb = align_up((size_t)(B * H * w.Sqp * w.DP) * 2, 256), kb = align_up((size_t)(B * Hkv * w.Skp * w.DP) * 2, 256);
  w.off_do16 = w.off_q16 + qb;
  w.off_k16 = w.off_do16 + qb;
  w.off_v16 = w.off_k16 + kb;
  const size_t pb = H > Hkv ? align_up((size_t)(B * H * Sk * D) * 4, 256) : 0;
  w.off_dkp = w.off_v16 + kb;
  w.off_dvp = w.off_dkp + pb;
  w.total = w.off_dvp + pb;
  return w;
}

template <int DP>
int launch_bwd_dp(const BwdParams& p, bool causal, bool has_bias, hipStream_t st) {
  dim3 g_kv((unsigned)(p.B * p.H), (unsigned)cdiv(p.Sk, 128));
  dim3 g_q((unsigned)(p.B * p.H), (unsigned)cdiv(p.Sq, 128));
#define LAUNCH(C, HB, DR)                                        \
  if constexpr (DP > 128) {                                      \
    dkdv_kernel<DP, C, HB, 1, DR><<<g_kv, NTH, 0, st>>>(p);      \
    TB_LAUNCH_CHECK("attn_bwd/dv");                              \
    dkdv_kernel<DP, C, HB, 2, DR><<<g_kv, NTH, 0, st>>>(p);      \
    TB_LAUNCH_CHECK("attn_bwd/dk");                              \
  } else {                                                       \
    dkdv_kernel<DP, C, HB, 0, DR><<<g_kv, NTH, 0, st>>>(p);      \
    TB_LAUNCH_CHECK("attn_bwd/dkdv");                            \
  }                                                              \
  dq_kernel<DP, C, HB, DR><<<g_q, NTH, 0, st>>>(p);              \
  TB_LAUNCH_CHECK("attn_bwd/dq");
  // the forms the kernels come in, then (GQA) the group sums of dK and dV
  if (p.drop_thr) {
    if (causal) {
      if (has_bias) { LAUNCH(true, true, true) } else { LAUNCH(true, false, true) }
    } else {
      if (has_bias) { LAUNCH(false, true, true) } else { LAUNCH(false, false, true) }
    }
  } else if (causal) {
    if (has_bias) { LAUNCH(true, true, false) } else { LAUNCH(true, false, false) }
  } else {
    if (has_bias) { LAUNCH(false, true, false) } else { LAUNCH(false, false, false) }
  }
#undef LAUNCH
  if (p.H > p.Hkv) {
    const int64_t per_head = (int64_t)p.Sk * p.D, n8 = (int64_t)p.B * p.Hkv * per_head / 8;
    const unsigned nb = (unsigned)cdiv(n8, NTH);
    kv_reduce_kernel<<<nb, NTH, 0, st>>>(p.dk_part, p.dk, p.H / p.Hkv, per_head, n8, p.gate);
    TB_LAUNCH_CHECK("attn_bwd/dk_reduce");
    kv_reduce_kernel<<<nb, NTH, 0, st>>>(p.dv_part, p.dv, p.H / p.Hkv, per_head, n8, p.gate);
    TB_LAUNCH_CHECK("attn_bwd/dv_reduce");
  }
  return 0;
}

}  // namespace

extern "C" size_t tbf16_attn_bwd_ws_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D) {
  return bwd_ws(B, H, Hkv, Sq, Sk, D).total;
}

extern "C" int tbf16_attn_bwd(const void* q, const void* k, const void* v, const void* o16, const float* lse,
                              const void* dout, const int32_t* exps_fwd, int64_t B, int64_t H, int64_t Hkv, int64_t Sq,
                              int64_t Sk, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                              const int64_t* v_strides, const int64_t* do_strides, const void* bias,
                              const int64_t* bias_strides, float scale, int causal, int t_do, float dropout_p,
                              uint64_t seed, void* dq, void* dk, void* dv, int32_t* exps_out, int32_t* overflow,
                              const int32_t* gate, void* ws, int64_t ws_bytes, void* stream) {
  TB_CHECK(B >= 0 && H > 0 && Hkv > 0 && Sq >= 0 && Sk >= 0 && H % Hkv == 0, "attn_bwd: bad shape");
  TB_CHECK(D > 0 && D % 8 == 0 && D <= 256, "attn_bwd: head dim must be a multiple of 8 up to 256");
  TB_CHECK(dropout_p >= 0.f && dropout_p < 1.f, "attn_bwd: dropout_p must be in [0, 1)");
  TB_CHECK(q && k && v && o16 && lse && dout && exps_fwd && dq && dk && dv && exps_out && overflow,
           "attn_bwd: null argument");
  TB_CHECK(q_strides && k_strides && v_strides && do_strides, "attn_bwd: strides missing");
  for (const int64_t* s : {q_strides, k_strides, v_strides, do_strides})
    TB_CHECK(s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0, "attn_bwd: strides must be multiples of 8");
  TB_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(dout) && aligned16(o16) && aligned16(dq) &&
               aligned16(dk) && aligned16(dv),
           "attn_bwd: tensors must be 16-byte aligned");
  if (bias) TB_CHECK(bias_strides != nullptr, "attn_bwd: bias strides missing");
  const BwdWs w = bwd_ws(B, H, Hkv, Sq, Sk, D);
  TB_CHECK(ws != nullptr && ws_bytes >= (int64_t)w.total, "attn_bwd: workspace too small");
  if (B == 0 || Sq == 0 || Sk == 0) return 0;
  hipStream_t st = as_stream(stream);
  float* part = reinterpret_cast<float*>(ws);
  // a gated attempt reuses the dO maxima its gate's attempt left in the workspace
  if (!gate) {
    if (int rc = launch_head_amax_partial(dout, TBF16_DT_BF16, B, H, Sq, D, do_strides[0], do_strides[1],
                                          do_strides[2], part, w.nch, st))
      return rc;
  }
  BwdParams p;
  p.q = (const uint16_t*)q; p.k = (const uint16_t*)k; p.v = (const uint16_t*)v;
  p.o16 = (const uint16_t*)o16; p.dout = (const uint16_t*)dout; p.lse = lse; p.exps_fwd = exps_fwd;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.d_sb = do_strides[0]; p.d_sh = do_strides[1]; p.d_ss = do_strides[2];
  p.bias = (const uint16_t*)bias;
  p.bias_sb = bias ? bias_strides[0] : 0; p.bias_sh = bias ? bias_strides[1] : 0; p.bias_sq = bias ? bias_strides[2] : 0;
  p.B = (int)B; p.H = (int)H; p.Hkv = (int)Hkv; p.Sq = (int)Sq; p.Sk = (int)Sk; p.D = (int)D;
  p.scale = scale; p.scale_log2 = scale * kLog2e; p.causal = causal; p.t_do = t_do;
  set_dropout(dropout_p, seed, p.drop_lo, p.drop_hi, p.drop_thr, p.drop_scale);
  p.part_do = part; p.nch_do = (int)w.nch;
  p.delta = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + w.off_delta);
  p.exps_out = exps_out; p.overflow = overflow; p.gate = gate;
  p.dq = (uint16_t*)dq; p.dk = (uint16_t*)dk; p.dv = (uint16_t*)dv;
  char* wsb = reinterpret_cast<char*>(ws);
  p.q16 = reinterpret_cast<uint16_t*>(wsb + w.off_q16);
  p.do16 = reinterpret_cast<uint16_t*>(wsb + w.off_do16);
  p.k16 = reinterpret_cast<uint16_t*>(wsb + w.off_k16);
  p.v16 = reinterpret_cast<uint16_t*>(wsb + w.off_v16);
  p.dk_part = H > Hkv ? reinterpret_cast<float*>(wsb + w.off_dkp) : nullptr;
  p.dv_part = H > Hkv ? reinterpret_cast<float*>(wsb + w.off_dvp) : nullptr;
  p.Sqp = (int)w.Sqp; p.Skp = (int)w.Skp; p.DPc = (int)w.DP;
  // q16, k16, v16 and e do not depend on t_do: a gated attempt finds them in the
  // workspace and exps_out, and its delta pass derives G
  if (!gate) {
    const int64_t rpb = NTH / (w.DP / 8);
    prep_kernel<<<dim3((unsigned)cdiv(std::max(w.Sqp, w.Skp), 4 * rpb), (unsigned)(B * H + 2 * B * Hkv)), NTH, 0, st>>>(p);
    TB_LAUNCH_CHECK("attn_bwd/prep");
  }
  delta_kernel<<<dim3((unsigned)cdiv(w.Sqp, 16), (unsigned)(B * H)), NTH, 0, st>>>(p);
  TB_LAUNCH_CHECK("attn_bwd/delta");
  if (D <= 64) return launch_bwd_dp<64>(p, causal != 0, bias != nullptr, st);
  if (D <= 128) return launch_bwd_dp<128>(p, causal != 0, bias != nullptr, st);
  return launch_bwd_dp<256>(p, causal != 0, bias != nullptr, st);
}
