// Scaled attention forward on CDNA4 fp16 MFMA (flash-style, no S x S buffer).
//
// Exponents (tbf16/attention.py:38-48), computed in each block's prologue from
// per-head partial maxima written by a memory-bound pre-pass:
//   eq = max_{b,h} frexp(amax q[b,h]), ek likewise, a = floor((ek - eq) / 2)
//   clamped to [ek - 14, 14 - eq], ev[b, hkv] = frexp(amax v[b, hkv]) - v_exp.
// A conversion pass (whose blocks also derive a and ev from those maxima) writes
// k16 = k * 2^-a and v16 = v * 2^-ev (exact powers of two) to the workspace as
// fp16, k16 row-major (B, Hkv, Skp, DP) and v16 transposed per 64-key tile
// (B, Hkv, Skp / 64, DP, 64: each tile's V^T one contiguous 2 * 64 * DP-byte
// block) with keys permuted as the PV operand wants them, both zero-padded, so the forward
// kernel copies K and V tiles global -> LDS directly (buffer_load ... lds, no
// registers in between): each K/V element is converted once instead of once per
// query block. q16 = q * 2^a is converted on the fly (once per
// row).
//
// Block = 4 or 8 waves, 32 query rows per wave; key tiles of 64.
//  - a wave keeps its 32 q rows as MFMA fragments in registers for the whole
//    kernel and computes S^T = K Q^T with v_mfma_f32_32x32x16_f16 (K from LDS), so
//    each lane owns ONE query row: row max / sum need one exchange with lane ^ 32.
//  - online softmax in fp32, base 2 (logit * scale * log2 e), P rounded to fp16.
//  - O^T = V^T P^T: V is stored transposed in LDS (d-major, keys permuted within
//    each 16-key group by swapping index bits 2 and 3) so that the A fragment of
//    a lane is one 16-byte read and P's fragment comes straight from S^T's
//    accumulators without any cross-lane shuffle.
//  - row sums l come from the fp16 P that enters the PV product (v_dot2 with
//    ones), so the normalisation matches the weights actually applied.
//  - output bf16(O / l * 2^ev) written from registers: one rounding.
// Causal blocks are launched heaviest first, or (few blocks per CU) each takes a
// heavy and a light query tile; key tiles past the diagonal are skipped, and
// only tiles crossing the diagonal or the end of the keys run the masked copy of
// the tile loop.
#include <stdlib.h>

#include <algorithm>
#include <math.h>

#include <type_traits>

#include "abi_util.h"
#include "common.h"

using namespace tbf16;

namespace tbf16 {
int64_t head_amax_chunks(int64_t BH, int64_t S);
}  // namespace tbf16

namespace {

constexpr int BKV = 64;
constexpr float kLog2e = 1.4426950408889634f;

struct FwdParams {
  const uint16_t *q, *k, *v;
  uint16_t *k16, *vt16;  // workspace copies: (B, Hkv, Skp, DP) and (B, Hkv, Skp / BKV, DP, BKV)
  int32_t* ex;           // workspace exponents {a, 0, ev[b * Hkv + hk]...}
  int Skp, DPc;
  int64_t q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss;
  const uint16_t* bias;
  int64_t bias_sb, bias_sh, bias_sq;
  int B, H, Hkv, Sq, Sk, D;
  float scale_log2;
  int v_exp;
  const float *part_q, *part_k, *part_v;
  int nch_q, nch_k, nch_v;
  uint16_t* o;
  float* lse;
  uint16_t* o16;
  int32_t* exps;
  int pair;  // causal: block x handles query tiles ntiles-1-x and x (balanced work per block)
  // conv_k: kv_prep writes k16 (else the forward reads k's bf16 rows directly);
  // derive_a: the q and k partial maxima exist and kv_prep derives a from them
  int conv_k, derive_a;
  // dropout (DROP kernels): keep iff the hashed 16-bit value >= drop_thr, kept
  // weights scaled by drop_scale = 1 / (1 - p)
  uint32_t drop_lo, drop_hi, drop_thr;
  float drop_scale;
};

__device__ __forceinline__ int perm16(int key) {  // swap bits 2 and 3 of a key index
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

template <int DP>
__device__ __forceinline__ int swz_k(int row, int chunk) {
  constexpr int RB = DP * 2;
  if constexpr (DP >= 128) return row * RB + ((chunk ^ (row & 15)) << 4);
  else return row * RB + ((chunk ^ ((row >> 1) & 7)) << 4);
}

__device__ __forceinline__ int swz_vt(int d, int chunk) { return d * 128 + ((chunk ^ ((d >> 1) & 7)) << 4); }

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// One 32x32x16 step of S^T = K Q^T: fp16 operands (k16, q 2^a), or with KBF the
// raw bf16 rows of k and q (v_mfma_f32_32x32x16_bf16, the same rate on gfx950).
// Scaling a bf16 value by 2^a into fp16 is exact unless it leaves fp16's normal
// range, so both forms multiply the same values: q.k 2^(a - a).
template <bool KBF>
__device__ __forceinline__ floatx16 mfma_qk(half8 k, half8 q, floatx16 c) {
  if constexpr (KBF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, k), __builtin_bit_cast(bf16x8, q), c, 0,
                                                    0, 0);
  else return __builtin_amdgcn_mfma_f32_32x32x16_f16(k, q, c, 0, 0, 0);
}

// Block-wide max of an int (NT threads, one slot per wave in red).
template <int NT>
__device__ __forceinline__ int block_max_int(int v, int* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) r = max(r, red[i]);
  return r;
}

// Masks the scores of a key tile that crosses the end of the keys or (causal)
// the diagonal: keys >= Sk or > qmax become -inf. Lane layout of S^T: key
// key0 + 32 kh + 8 (r / 4) + 4 fk + r % 4 in accumulator r of half kh. Called
// from a wave-uniform branch, so interior tiles skip it.
__device__ __forceinline__ void mask_tile(floatx16 (&sacc)[2], int key0, int Sk, int qmax, int fk) {
  const int lim = min(Sk - 1, qmax) - key0 - 4 * fk;  // keep offsets <= lim
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (kh * 32 + 8 * (r >> 2) + (r & 3) > lim) sacc[kh][r] = -INFINITY;
}

// Halves j of four rows (packed fp16 words w0..w3 holding halves 2i, 2i+1) -> the
// 4-key run {r0[j], r1[j], r2[j], r3[j]} as two dwords, with v_perm_b32.
__device__ __forceinline__ uint2 gather4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, bool odd) {
  const uint32_t sel = odd ? 0x07060302u : 0x05040100u;
  return make_uint2(__builtin_amdgcn_perm(w1, w0, sel), __builtin_amdgcn_perm(w3, w2, sel));
}

// Exponents (tbf16/attention.py:38-48) from the per-head partial maxima, once:
// a and ev[b * Hkv + hk] into the workspace (and into the caller's exps if given).
// Per-head maxima of the partials, wave-parallel: wave w reduces heads w, w + 4,
// ... (a lane per chunk), eight heads' loads in flight before any is reduced.
// Calls f(head, max) on lane 0 of the reducing wave.
template <typename F>
__device__ __forceinline__ void heads_max(const float* part, int nbh, int nch, F f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int bh0 = wave; bh0 < nbh; bh0 += 32) {
    float m[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = 0.f;
    for (int c = lane; c < nch; c += 64) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int bh = bh0 + 4 * j;
        if (bh < nbh) m[j] = fmaxf(m[j], part[bh * nch + c]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int bh = bh0 + 4 * j;
      const float mx = wave_max(m[j]);
      if (bh < nbh && lane == 0) f(bh, mx);
    }
  }
}

// k16 and the permuted v16^T for one 64-key tile of one (batch, kv head): block
// (tile, b * Hkv + hk), 256 threads. K: thread t converts 16-byte chunks t + 256 i
// (row c / (DP / 8), chunk c % (DP / 8)). V: thread t takes blocks t + 256 i of 4
// keys x 8 columns (kg = block % 16, dc = block / 16), converts the four 16-byte
// row pieces and writes, for each of its 8 columns d, the 4-key run at position
// perm16(4 kg) of row d of the tile's V^T block (8 bytes; the 16 threads of one dc
// fill each 128-byte row; the tile's DP rows are one contiguous block, which the
// forward kernel then copies to LDS 1 KB at a time). Keys past Sk and columns
// past D are written as zeros.
// Each block also derives the exponents (tbf16/attention.py:38-48) from the
// per-head partial maxima: a from all q and k heads, ev of its own kv head;
// when the forward reads k's bf16 rows itself (conv_k = 0) no k16 is written,
// and a only where the caller asks for the exponents (derive_a);
// blocks (0, bhk) store them (a by block (0, 0)) to the workspace and to the
// caller's exps, where the forward kernel and the backward read them.
template <int DP>
__global__ __launch_bounds__(256) void kv_prep_kernel(FwdParams p) {
  constexpr int CPR = DP / 8;
  constexpr int NKL = BKV * CPR / 256;         // K chunks per thread
  constexpr int NVB = (16 * CPR + 255) / 256;  // V blocks of 4 keys x 8 columns per thread
  __shared__ int red[4];
  const int bhk = blockIdx.y, b = bhk / p.Hkv, hk = bhk % p.Hkv;
  const int key0 = blockIdx.x * BKV;
  const uint16_t* kb = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const uint16_t* vb = p.v + (int64_t)b * p.v_sb + (int64_t)hk * p.v_sh;
  // The raw tiles are loaded first (they do not depend on the exponents), so they
  // are in flight together with the partial-maxima loads of the exponent
  // derivation below; its first block barrier waits for both.
  uint4 kr[NKL], vr[NVB][4];
  if (p.conv_k) {
#pragma unroll
    for (int i = 0; i < NKL; ++i) {
      const int c = threadIdx.x + i * 256, row = c / CPR, ch = c % CPR;
      const int key = key0 + row;
      kr[i] = key < p.Sk && ch * 8 < p.D ? ldg16(kb + (int64_t)key * p.k_ss + ch * 8) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int blk = threadIdx.x + i * 256;
    const int kg = blk & 15, dc = blk >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + 4 * kg + r;
      vr[i][r] = blk < 16 * CPR && key < p.Sk && dc * 8 < p.D ? ldg16(vb + (int64_t)key * p.v_ss + dc * 8)
                                                              : make_uint4(0, 0, 0, 0);
    }
  }
  // a (tbf16/attention.py:44-45) where q's and k's maxima were taken (the caller
  // asked for the exponents, or k16 is written) and this block needs it: every
  // block that converts K, else only block (0, 0), which stores it; else 0, unused
  int a = 0;
  if (p.derive_a && (p.conv_k || (blockIdx.x == 0 && bhk == 0))) {
    int eq = INT_MIN, ek = INT_MIN;
    heads_max(p.part_q, p.B * p.H, p.nch_q, [&](int, float m) { eq = max(eq, frexp_exp(m)); });
    heads_max(p.part_k, p.B * p.Hkv, p.nch_k, [&](int, float m) { ek = max(ek, frexp_exp(m)); });
    eq = block_max_int<256>(eq, red);
    ek = block_max_int<256>(ek, red);
    a = (ek - eq) >> 1;  // floor division
    a = max(min(a, 14 - eq), ek - 14);
  }
  float mv = 0.f;
  for (int c = threadIdx.x; c < p.nch_v; c += 256) mv = fmaxf(mv, p.part_v[bhk * p.nch_v + c]);
  mv = wave_max(mv);
  __syncthreads();  // red is reused
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = __float_as_int(mv);  // non-negative: int order = float order
  __syncthreads();
  const int ev = frexp_exp(__int_as_float(max(max(red[0], red[1]), max(red[2], red[3])))) - p.v_exp;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    p.ex[2 + bhk] = ev;
    if (p.exps) p.exps[2 + bhk] = ev;
    if (bhk == 0) {
      p.ex[0] = a;
      p.ex[1] = 0;
      if (p.exps) {
        p.exps[0] = a;
        p.exps[1] = 0;
      }
    }
  }
  const float sk = ldexp1(-a), sv = ldexp1(-ev);
  uint16_t* k16 = p.k16 + ((int64_t)bhk * p.Skp + key0) * DP;
  uint16_t* vt16 = p.vt16 + ((int64_t)bhk * p.Skp + key0) * DP;  // this tile's (DP, BKV) block
  if (p.conv_k) {
#pragma unroll
    for (int i = 0; i < NKL; ++i) {
      const int c = threadIdx.x + i * 256, row = c / CPR, ch = c % CPR;
      stg16(k16 + row * DP + ch * 8, cvt_bf16x8_f16x8(kr[i], sk));
    }
  }
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int blk = threadIdx.x + i * 256;
    if (blk >= 16 * CPR) break;
    const int kg = blk & 15, dc = blk >> 4;
    uint4 cv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) cv[r] = cvt_bf16x8_f16x8(vr[i][r], sv);
    const int pos = perm16(4 * kg);
    const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&cv[0]);
    const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&cv[1]);
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&cv[2]);
    const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&cv[3]);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<uint2*>(vt16 + (dc * 8 + j) * BKV + pos) =
          gather4(w0[j >> 1], w1[j >> 1], w2[j >> 1], w3[j >> 1], j & 1);
  }
}

// Forward kernel: NW waves, 32 query rows each (BQ = 32 * NW), 64-key tiles
// staged in two LDS stages by direct global -> LDS loads shared out over all
// waves. NW = 8: two waves per SIMD, one block per CU; NW = 4: two blocks per CU.
// SPLIT (NW = 8): waves w and w + 4 take the same 32 query rows (BQ = 128) and
// the even and the odd key tiles respectively, from four LDS stages (a pair of
// tiles in flight while the other pair is read); the odd group hands its O^T,
// running max and row sums to its partner through LDS at the end. A causal grid
// of few blocks then gets both the heavy/light pairing (every block the same
// work) and two waves per SIMD.
// KBF: S^T = K Q^T on the raw bf16 rows of k and q (bf16 MFMA), K tiles copied
// straight from k (head dim = DP); only V goes through the conversion pass.
template <int DP, int NW, bool CAUSAL, bool HAS_BIAS, bool DROP, bool SPLIT = false, bool KBF = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(DP > 128 ? 1 : 2, DP > 128 ? 1 : 2))) void
attn_fwd_kernel(FwdParams p) {
  static_assert(!SPLIT || (NW == 8 && DP <= 128 && !HAS_BIAS && !DROP), "split-key blocks: 8 waves, no bias or dropout");
  static_assert(!KBF || (DP <= 128 && !HAS_BIAS && !DROP), "bf16 K rows: head dim <= 128, no bias or dropout");
  constexpr int RB = SPLIT ? NW / 2 : NW;  // 32-row query blocks per block
  constexpr int NT = NW * 64, BQW = 32 * RB;
  constexpr int KS = DP / 16;            // MFMA k-steps over the head dim
  constexpr int DB = DP / 32;            // 32-wide d blocks of O^T
  constexpr int CPR = DP / 8;            // 16-byte chunks per K row
  constexpr int KBYTES = BKV * DP * 2;
  constexpr int STAGE = KBYTES + DP * 128;
  // V^T fragments read during the QK product (registers allow it up to DP = 128
  // without the bias rows or the dropout hashing)
  constexpr bool VPRE = DP <= 128 && !HAS_BIAS && !DROP;
  // K and V^T tiles go global -> LDS directly, 1 KB per wave instruction: BPW
  // such blocks per wave per tile, the first KPW of them K, the rest V^T
  constexpr int KBLK = KBYTES / 1024, NBLK = STAGE / 1024;
  static_assert(NBLK % NW == 0 && KBLK % NW == 0, "K/V staging blocks");
  constexpr int BPW = NBLK / NW, KPW = KBLK / NW;
  // two stages as separate objects, so that the compiler's LDS alias analysis
  // sees that reads of one stage never wait for the loads into the other (a
  // third stage, loads two tiles ahead, measured no faster)
  __shared__ __align__(1024) uint8_t smem0[STAGE];
  __shared__ __align__(1024) uint8_t smem1[STAGE];
  __shared__ __align__(1024) uint8_t smem2[SPLIT ? STAGE : 16];
  __shared__ __align__(1024) uint8_t smem3[SPLIT ? STAGE : 16];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fk = lane >> 5;
  const int rw = SPLIT ? wave % RB : wave;  // this wave's 32-row query block
  const int grp = SPLIT ? wave / RB : 0;    // SPLIT: key tiles of this parity
  // grid (heads, query blocks): dispatch runs over heads first, so the heaviest
  // query blocks of every head (causal) go out before any lighter one
  const int bh = blockIdx.x, b = bh / p.H, h = bh % p.H;
  const int hk = h / (p.H / p.Hkv);

  // ---- exponents (derived by kv_prep_kernel) ----
  const int a = p.ex[0];
  const int ev = p.ex[2 + b * p.Hkv + hk];
  const float sq = ldexp1(a);

  // Query tiles of this block: one, or with pair (causal) the heavy tile
  // ntiles-1-x and then the light tile x, so every block does the same work.
  const int ntiles = (p.Sq + BQW - 1) / BQW;
  const int bx = (int)blockIdx.y;
  const int npass = (CAUSAL && p.pair) ? (bx == ntiles - 1 - bx ? 1 : 2) : 1;
  for (int pass = 0; pass < npass; ++pass) {
    const int qt = !CAUSAL ? bx : p.pair ? (pass == 0 ? ntiles - 1 - bx : bx) : (int)gridDim.y - 1 - bx;
    const int q0 = qt * BQW;
    // ---- Q fragments in registers (fp16, scaled by 2^a) ----
    const int qrow = q0 + rw * 32 + fr;
    const uint32_t drow = DROP ? drop_row((uint32_t)bh * (uint32_t)p.Sq + (uint32_t)qrow, p.drop_lo) : 0u;
    half8 qf[KS];
    {
      const uint16_t* qp = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)min(qrow, p.Sq - 1) * p.q_ss;
  #pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int d = 16 * s + 8 * fk;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (qrow < p.Sq && d < p.D) v = KBF ? ldg16(qp + d) : cvt_bf16x8_f16x8(ldg16(qp + d), sq);
        qf[s] = __builtin_bit_cast(half8, v);
      }
    }

    // ---- K / V^T staging: the workspace's converted tiles copied global -> LDS ----
    // Lane j of a wave instruction lands at byte 16 j of its 1 KB block, so the
    // row swizzle is applied on the source side: the lane fetches the logical
    // chunk that belongs at its LDS position. Block bi of a stage: K rows
    // (bi * 1024 / (2 DP) ...) for bi < KBLK, else V^T rows d.
    const int bhk = b * p.Hkv + hk;
    const BufRes kres = make_res(p.k16 + (int64_t)bhk * p.Skp * DP, min<int64_t>((int64_t)p.Skp * DP * 2, 0x7fffffff));
    // KBF: k's own rows, stride k_ss; each tile gets a resource that starts at its
    // first key and ends at the last key's last element, so rows past Sk read
    // zeros (the range check covers the VGPR offset, not the SGPR one)
    const uint16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
    const int krow = KBF ? (int)p.k_ss : DP;  // elements from one K row to the next
    const BufRes vres = make_res(p.vt16 + (int64_t)bhk * DP * p.Skp, min<int64_t>((int64_t)DP * p.Skp * 2, 0x7fffffff));
    int voff[BPW];
  #pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int bi = wave + NW * i;
      if (i < KPW) {
        const int byte = bi * 1024 + 16 * lane, row = byte / (2 * DP), phys = (byte % (2 * DP)) >> 4;
        const int lch = (swz_k<DP>(row, phys) - row * 2 * DP) >> 4;  // the XOR swizzle is its own inverse
        voff[i] = (row * krow + lch * 8) * 2;
      } else {
        const int byte = (bi - KBLK) * 1024 + 16 * lane, d = byte >> 7, phys = (byte & 127) >> 4;
        const int ch = (swz_vt(d, phys) - d * 128) >> 4;
        voff[i] = (d * BKV + ch * 8) * 2;
      }
    }
    auto dload = [&](uint8_t* stage, int kb) {
      const uint32_t base = lds_addr(stage);
      // (32-bit scalar arithmetic: the tile's last row is at most BKV - 1 rows on,
      // and the launcher keeps BKV rows of k within 2^31 bytes; 64-bit forms
      // compile to vector code and a waterfall loop around every load)
      const int last = min(p.Sk - 1 - kb * BKV, BKV - 1);
      const BufRes ktile = KBF ? make_res(kbase + (int64_t)kb * BKV * p.k_ss, (last * krow + p.D) * 2) : kres;
      const int ksoff = KBF ? 0 : kb * BKV * DP * 2;
  #pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const uint32_t dst = base + (wave + NW * i) * 1024;
        if (i < KPW) buf_load16_lds(ktile, dst, voff[i], ksoff);
        else buf_load16_lds(vres, dst, voff[i], kb * BKV * DP * 2);
      }
    };

    floatx16 acc_o[DB];
  #pragma unroll
    for (int i = 0; i < DB; ++i)
  #pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[i][r] = 0.f;
    // running max in log2 units; stays stale until a row's max grows by more than
    // 2^8, so exp2 arguments are <= 8 and P <= 256 (fp16-safe)
    float m_run = -INFINITY, l_run = 0.f;
    const float c = HAS_BIAS ? 1.f : p.scale_log2;

    const int nkb_all = (p.Sk + BKV - 1) / BKV;
    int nkb = nkb_all;
    if constexpr (CAUSAL) nkb = min(nkb_all, (min(q0 + BQW, p.Sq) + BKV - 1) / BKV);
    const uint16_t* brow = nullptr;
    if constexpr (HAS_BIAS)
      brow = p.bias + (int64_t)b * p.bias_sb + (int64_t)h * p.bias_sh + (int64_t)min(qrow, p.Sq - 1) * p.bias_sq;

    // The last PV step of each tile runs at the start of the next tile, after its
    // first K reads have gone out (its fragments were read before the barrier),
    // so the barrier's drain and those reads' latency hide behind 4 MFMAs. It
    // starts as zeros (adds nothing) and is flushed after the last tile.
    half8 dpf, dvf[DB];
    for (int e = 0; e < 8; ++e) dpf[e] = (_Float16)0.f;
  #pragma unroll
    for (int db = 0; db < DB; ++db) dvf[db] = dpf;
    auto deferred = [&]() {
  #pragma unroll
      for (int db = 0; db < DB; ++db) acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(dvf[db], dpf, acc_o[db], 0, 0, 0);
    };
    auto step = [&](int kb, const uint8_t* sK, auto masked_c) {
      constexpr bool MASKED = decltype(masked_c)::value;
      const uint8_t* sV = sK + KBYTES;
      // S^T = K Q^T for two 32-key halves: lane = one query row, 16 keys each.
      // Fragment reads run ahead of their MFMAs (the compiler otherwise reads each
      // fragment at its use and waits on it): the first half's K fragments, then
      // the second half's K fragments between the first half's MFMAs, then the V^T
      // fragments of the first two PV steps between the second half's MFMAs; the
      // remaining V^T fragments are read during the PV MFMAs two steps ahead.
      // Pinned by instruction-group schedules (DP <= 128 without bias rows; else
      // each fragment is read at its use).
      floatx16 sacc[2];
  #pragma unroll
      for (int kh = 0; kh < 2; ++kh)
  #pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kh][r] = 0.f;
      auto kread = [&](int kh, int s) {
        return *reinterpret_cast<const half8*>(sK + swz_k<DP>(kh * 32 + fr, 2 * s + fk));
      };
      auto vread = [&](int ks, int db) {
        return *reinterpret_cast<const half8*>(sV + swz_vt(db * 32 + fr, 2 * ks + fk));
      };
      half8 vf[VPRE ? 4 : 1][DB];
      if constexpr (VPRE) {
        // One read queue: the K fragments in MFMA order, the two halves' chains
        // alternating (consecutive MFMAs never depend on each other: a dependent
        // MFMA waits for its predecessor's result), then the V^T fragments of PV
        // steps 0 and 1; reads run LA MFMAs ahead, two per MFMA at first.
        constexpr int LA = 4, NK = 2 * KS, NQ = NK + 2 * DB, EXTRA = NQ - LA - NK;
        static_assert(EXTRA >= 0 && EXTRA <= NK, "read queue");
        half8 fq[NQ];
  #pragma unroll
        for (int j = 0; j < NQ; ++j) {
          if (j < NK) fq[j] = kread(j & 1, j >> 1);
          else fq[j] = vread((j - NK) / DB, (j - NK) % DB);
        }
        deferred();
  #pragma unroll
        for (int j = 0; j < NK; ++j)
          sacc[j & 1] = mfma_qk<KBF>(fq[j], qf[j >> 1], sacc[j & 1]);
  #pragma unroll
        for (int ks = 0; ks < 2; ++ks)
  #pragma unroll
          for (int db = 0; db < DB; ++db) vf[ks][db] = fq[NK + ks * DB + db];
        __builtin_amdgcn_sched_group_barrier(0x100, LA, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, DB, 0);  // the previous tile's deferred step
  #pragma unroll
        for (int i = 0; i < EXTRA; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
  #pragma unroll
        for (int i = EXTRA; i < NK; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      } else {
        deferred();
  #pragma unroll
        for (int s = 0; s < KS; ++s)
  #pragma unroll
          for (int kh = 0; kh < 2; ++kh) sacc[kh] = mfma_qk<KBF>(kread(kh, s), qf[s], sacc[kh]);
      }
      const int key0 = kb * BKV;
      const bool edge = (key0 + BKV > p.Sk) || (CAUSAL && key0 + BKV - 1 > q0 + rw * 32);
      if constexpr (HAS_BIAS) {
  #pragma unroll
        for (int kh = 0; kh < 2; ++kh)
  #pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = key0 + kh * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
            sacc[kh][r] = sacc[kh][r] * p.scale_log2 +
                          (key < p.Sk ? (float)__builtin_bit_cast(_Float16, brow[key]) * kLog2e : 0.f);
          }
      }
      if (MASKED && edge) mask_tile(sacc, key0, p.Sk, CAUSAL ? qrow : INT_MAX, fk);
      float mx = -INFINITY;
  #pragma unroll
      for (int kh = 0; kh < 2; ++kh)
  #pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kh][r]);
      mx = max_xor32(mx) * c;
      if (__any(mx > m_run + 8.f)) {  // wave-uniform: rescale O and l only when some row needs it
        const float m_new = fmaxf(m_run, mx);
        const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
  #pragma unroll
        for (int i = 0; i < DB; ++i)
  #pragma unroll
          for (int r = 0; r < 16; ++r) acc_o[i][r] *= alpha;
      }
      const float mneg = (m_run == -INFINITY) ? 0.f : -m_run;
      // row sums from the fp16 P that the PV product uses (v_dot2 with ones)
      const half2v ones = {(_Float16)1.f, (_Float16)1.f};
      float lsum = 0.f;
      uint32_t pk[2][8];
  #pragma unroll
      for (int kh = 0; kh < 2; ++kh)
  #pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[kh][r], c, mneg));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[kh][r + 1], c, mneg));
          pk[kh][r >> 1] = pack_f16(p0, p1);
          lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, pk[kh][r >> 1]), ones, lsum, false);
          if constexpr (DROP) {  // l keeps the undropped weights; the PV product gets the kept ones,
            // unscaled (P reaches 2^8 under the lazy rescale: P / (1 - p) would leave fp16
            // for p near 1), and the epilogue applies 1 / (1 - p) in fp32
            const int key = key0 + kh * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);  // even
            const uint32_t u = drop_pair(drow, key, p.drop_hi);
            pk[kh][r >> 1] = pack_f16(drop_keep(u, key, p.drop_thr) ? p0 : 0.f,
                                      drop_keep(u, key + 1, p.drop_thr) ? p1 : 0.f);
          }
        }
      l_run += lsum;
      // O^T += V^T P^T over four 16-key steps
  #pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint4 pw = make_uint4(pk[ks >> 1][4 * (ks & 1) + 0], pk[ks >> 1][4 * (ks & 1) + 1],
                                    pk[ks >> 1][4 * (ks & 1) + 2], pk[ks >> 1][4 * (ks & 1) + 3]);
        const half8 pf = __builtin_bit_cast(half8, pw);
        if (ks == 3) {  // deferred past the barrier (operands stay in registers)
          dpf = pf;
  #pragma unroll
          for (int db = 0; db < DB; ++db) {
            if constexpr (VPRE) dvf[db] = vf[3][db];
            else dvf[db] = vread(3, db);
          }
        } else if constexpr (VPRE) {
  #pragma unroll
          for (int db = 0; db < DB; ++db) {
            acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[ks][db], pf, acc_o[db], 0, 0, 0);
            if (ks < 2) vf[ks + 2][db] = vread(ks + 2, db);
          }
        } else {
  #pragma unroll
          for (int db = 0; db < DB; ++db) acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vread(ks, db), pf, acc_o[db], 0, 0, 0);
        }
      }
    };

    // Tile kb lives in stage kb % 2; tile kb + 1's loads go out when tile kb's
    // computation starts (its stage was last read before the previous barrier)
    // and are waited for at the barrier that ends tile kb. Tiles [0, nfull) are
    // whole for every wave of the block; the rest (the diagonal, the end of the
    // keys) run in a second loop with the masking compiled in (nfull is even, so
    // both loops start on stage 0).
    int nfull = min(nkb, p.Sk / BKV);
    if constexpr (CAUSAL) nfull = min(nfull, (q0 + 1) / BKV);
    if constexpr (SPLIT) {
      // Super-tile j = tiles 2 j (group 0) and 2 j + 1 (group 1) in stage pair
      // j % 2; the other pair's two loads go out when super-tile j's computation
      // starts. Super-tiles [0, nfs) are whole for every wave (nfs even, so both
      // loops start on stage pair 0); a group with no tile in the last super-tile
      // still takes part in its loads and barrier.
      const int nsup = (nkb + 1) / 2, nfs = (nfull / 2) & ~1;
      auto supers = [&](int j_begin, int j_end, auto masked_c) {
        auto one = [&](int j, const uint8_t* c0, const uint8_t* c1, uint8_t* n0, uint8_t* n1) {
          if (2 * j + 2 < nkb) dload(n0, 2 * j + 2);
          if (2 * j + 3 < nkb) dload(n1, 2 * j + 3);
          if (2 * j + grp < nkb) step(2 * j + grp, grp ? c1 : c0, masked_c);
          wait_vmem();
          __syncthreads();
        };
        for (int j = j_begin; j < j_end; j += 2) {
          one(j, smem0, smem1, smem2, smem3);
          if (j + 1 < j_end) one(j + 1, smem2, smem3, smem0, smem1);
        }
      };
      if (nkb > 0) dload(smem0, 0);
      if (nkb > 1) dload(smem1, 1);
      wait_vmem();
      __syncthreads();
      supers(0, nfs, std::false_type{});
      supers(nfs, nsup, std::true_type{});
    } else {
      nfull &= ~1;
      auto tiles = [&](int kb_begin, int kb_end, auto masked_c) {
        // tile kb from stage cur; tile kb + 1 loads into stage nxt
        auto one = [&](int kb, const uint8_t* cur, uint8_t* nxt) {
          if (kb + 1 < nkb) dload(nxt, kb + 1);
          step(kb, cur, masked_c);
          wait_vmem();
          __syncthreads();
        };
        for (int kb = kb_begin; kb < kb_end; kb += 2) {
          one(kb, smem0, smem1);
          if (kb + 1 < kb_end) one(kb + 1, smem1, smem0);
        }
      };
      if (nkb > 0) dload(smem0, 0);
      wait_vmem();
      __syncthreads();
      // (without the fragment prefetch, one loop with the masking branch keeps the
      // register allocation within bounds)
      if constexpr (VPRE) tiles(0, nfull, std::false_type{});
      tiles(VPRE ? nfull : 0, nkb, std::true_type{});
    }
    deferred();

    if constexpr (SPLIT) {
      // Group 1's partial O^T (lane-major, DB x 16 values per lane), running max
      // and row sums go through the idle stages; group 0 merges them into its own:
      // m = max(m0, m1), O = O0 2^(m0 - m) + O1 2^(m1 - m), l likewise.
      float* xo = reinterpret_cast<float*>(rw < 2 ? smem0 : smem1) + (rw & 1) * (DB * 16 * 64);
      float* xm = reinterpret_cast<float*>(smem2) + rw * 128;
      if (grp) {
  #pragma unroll
        for (int db = 0; db < DB; ++db)
  #pragma unroll
          for (int r = 0; r < 16; ++r) xo[(db * 16 + r) * 64 + lane] = acc_o[db][r];
        xm[lane] = m_run;
        xm[64 + lane] = l_run;
      }
      __syncthreads();
      if (!grp) {
        const float m1 = xm[lane], l1 = xm[64 + lane];
        const float mm = fmaxf(m_run, m1);
        const float a0 = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mm);
        const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mm);
        m_run = mm;
        l_run = l_run * a0 + l1 * a1;
  #pragma unroll
        for (int db = 0; db < DB; ++db)
  #pragma unroll
          for (int r = 0; r < 16; ++r) acc_o[db][r] = acc_o[db][r] * a0 + xo[(db * 16 + r) * 64 + lane] * a1;
      }
      __syncthreads();  // the next pass reloads the stages
    }

    // ---- epilogue ----
    const float l_tot = sum_xor32(l_run);
    if ((!SPLIT || grp == 0) && qrow < p.Sq) {
    const float sev = ldexp1(ev);
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
          y[e] = l_tot > 0.f ? acc_o[db][4 * rq + e] / l_tot : 0.f;
          if constexpr (DROP) y[e] *= p.drop_scale;
        }
        *reinterpret_cast<uint2*>(p.o + orow + d) =
            make_uint2(pack_bf16(y[0] * sev, y[1] * sev), pack_bf16(y[2] * sev, y[3] * sev));
        if (p.o16) *reinterpret_cast<uint2*>(p.o16 + orow + d) = make_uint2(pack_f16(y[0], y[1]), pack_f16(y[2], y[3]));
      }
    // lse in log2 units (v_log_f32); rows that see no key get +inf so the
    // backward's exp2(logit - lse) is 0 there
    if (p.lse && fk == 0)
      p.lse[(int64_t)bh * p.Sq + qrow] = (l_tot > 0.f) ? m_run + __builtin_amdgcn_logf(l_tot) : INFINITY;
    }
  }
}

struct WsLayout {
  int64_t nch_q, nch_k, nch_v, Skp, DP;
  size_t off_k, off_v, off_ex, off_k16, off_vt16, total;
};

// partial maxima of q | k | v, exponents {a, 0, ev...}, k16 (B, Hkv, Skp, DP),
// v16^T per key tile (B, Hkv, Skp / 64, DP, 64); Skp = Sk rounded up to the 64-key tile
WsLayout fwd_ws(int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D) {
  WsLayout w;
  w.nch_q = head_amax_chunks(B * H, Sq);
  w.nch_k = head_amax_chunks(B * Hkv, Sk);
  w.nch_v = w.nch_k;
  w.Skp = cdiv(Sk, BKV) * BKV;
  w.DP = D <= 64 ? 64 : D <= 128 ? 128 : 256;
  const size_t bq = align_up((size_t)(B * H * w.nch_q) * 4, 256), bk = align_up((size_t)(B * Hkv * w.nch_k) * 4, 256);
  const size_t bkv = align_up((size_t)(B * Hkv * w.Skp * w.DP) * 2, 256);
  w.off_k = bq;
  w.off_v = bq + bk;
  w.off_ex = bq + 2 * bk;
  w.off_k16 = w.off_ex + align_up((size_t)(2 + B * Hkv) * 4, 256);
  w.off_vt16 = w.off_k16 + bkv;
  w.total = w.off_vt16 + bkv;
  return w;
}

template <int DP, int NW>
int launch_fwd_nw(const FwdParams& p, bool causal, bool has_bias, bool split, dim3 grid, hipStream_t st) {
  // dropout kernels exist for 4-wave blocks only (the launcher picks those)
  if (p.drop_thr) {
    if constexpr (NW == 4) {
      if (causal) {
        if (has_bias) attn_fwd_kernel<DP, 4, true, true, true><<<grid, 256, 0, st>>>(p);
        else attn_fwd_kernel<DP, 4, true, false, true><<<grid, 256, 0, st>>>(p);
      } else {
        if (has_bias) attn_fwd_kernel<DP, 4, false, true, true><<<grid, 256, 0, st>>>(p);
        else attn_fwd_kernel<DP, 4, false, false, true><<<grid, 256, 0, st>>>(p);
      }
    }
  } else if (split) {
    if constexpr (NW == 8 && DP <= 128) {
      if (!p.conv_k) attn_fwd_kernel<DP, 8, true, false, false, true, true><<<grid, 512, 0, st>>>(p);
      else attn_fwd_kernel<DP, 8, true, false, false, true><<<grid, 512, 0, st>>>(p);
    }
  } else if (!p.conv_k) {  // bf16 K rows (no bias rows, no dropout, head dim <= 128)
    if constexpr (DP <= 128) {
      if (causal) attn_fwd_kernel<DP, NW, true, false, false, false, true><<<grid, NW * 64, 0, st>>>(p);
      else attn_fwd_kernel<DP, NW, false, false, false, false, true><<<grid, NW * 64, 0, st>>>(p);
    }
  } else if (causal) {
    if (has_bias) attn_fwd_kernel<DP, NW, true, true, false><<<grid, NW * 64, 0, st>>>(p);
    else attn_fwd_kernel<DP, NW, true, false, false><<<grid, NW * 64, 0, st>>>(p);
  } else {
    if (has_bias) attn_fwd_kernel<DP, NW, false, true, false><<<grid, NW * 64, 0, st>>>(p);
    else attn_fwd_kernel<DP, NW, false, false, false><<<grid, NW * 64, 0, st>>>(p);
  }
  TB_LAUNCH_CHECK("attn_fwd");
  return 0;
}

// 8-wave blocks (256 queries, two waves per SIMD) share each K/V tile between
// more queries and win once there are enough of them: measured on MI355X
// (causal, D = 128) at S = 16384, B = 1, H = 16 (1024 blocks of 8 waves, 962 vs
// 925 TFLOPS) and at S = 4096, B = 2, H = 16 (512 blocks, 632 vs 611). With at
// most ~1.5 rounds of 8-wave blocks a causal grid is better served by 4-wave
// blocks that pair a heavy and a light query tile (S = 4096, B = 1: 563 vs 476).
// Head dim 256 always uses 4-wave blocks (one wave per SIMD, 512 registers).
template <int DP>
int launch_fwd_dp(FwdParams p, bool causal, bool has_bias, hipStream_t st, int nw_override) {
  const int64_t tiles8 = cdiv(p.Sq, 256) * p.B * p.H, tiles4 = cdiv(p.Sq, 128) * p.B * p.H;
  // causal with few blocks: 4-wave blocks that pair a heavy and a light query
  // tile, so every block has the same work (heaviest-first ordering only
  // balances many rounds); otherwise as measured above
  const bool pair = causal && tiles4 >= 2 * p.B * p.H && tiles8 < 384 && nw_override <= 0 &&
                    getenv("TBF16_ATTN_NOPAIR") == nullptr;
  // the paired grid runs as split-key 8-wave blocks where those exist (no bias
  // rows, no dropout, head dim <= 128); TBF16_ATTN_SPLIT=0 / 1 turns that off / on
  // for any causal grid (benchmarking)
  const char* sv = getenv("TBF16_ATTN_SPLIT");
  const bool split_ok = causal && DP <= 128 && !has_bias && !p.drop_thr && nw_override <= 0;
  const bool split = split_ok && (sv ? atoi(sv) != 0 : pair);
  int nw = nw_override > 0 ? nw_override : pair ? 4 : (tiles8 >= 128 ? 8 : 4);
  if (DP > 128 || p.drop_thr) nw = 4;
  if (split) nw = 8;
  const int64_t ntiles = cdiv(p.Sq, nw == 8 && !split ? 256 : 128);
  p.pair = pair && (nw == 4 || split);
  const dim3 grid(p.B * p.H, (unsigned)(p.pair ? cdiv(ntiles, 2) : ntiles));
  if (nw == 8) {
    if constexpr (DP <= 128) return launch_fwd_nw<DP, 8>(p, causal, has_bias, split, grid, st);
  }
  return launch_fwd_nw<DP, 4>(p, causal, has_bias, false, grid, st);
}

int check_bhsd(const char* fn, const char* name, const void* x, const int64_t* st, int64_t D) {
  TB_CHECK(x != nullptr && st != nullptr, "%s: %s missing", fn, name);
  TB_CHECK(aligned16(x) && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0,
           "%s: %s must be (B, H, S, D) with contiguous D %% 8 == 0, 16-byte aligned", fn, name);
  (void)D;
  return 0;
}

}  // namespace

extern "C" size_t tbf16_attn_fwd_ws_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D) {
  return fwd_ws(B, H, Hkv, Sq, Sk, D).total;
}

extern "C" int tbf16_attn_fwd(const void* q, const void* k, const void* v, int64_t B, int64_t H, int64_t Hkv,
                              int64_t Sq, int64_t Sk, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                              const int64_t* v_strides, const void* bias, const int64_t* bias_strides, float scale,
                              int causal, int v_exp, float dropout_p, uint64_t seed, void* o, float* lse, void* o16,
                              int32_t* exps, void* ws, int64_t ws_bytes, void* stream) {
  TB_CHECK(B >= 0 && H > 0 && Hkv > 0 && Sq >= 0 && Sk >= 0, "attn_fwd: bad shape");
  TB_CHECK(H % Hkv == 0, "attn_fwd: query heads must be a multiple of key/value heads");
  TB_CHECK(D > 0 && D % 8 == 0 && D <= 256, "attn_fwd: head dim must be a multiple of 8 up to 256");
  TB_CHECK(B * H < (int64_t)1 << 31 && Sq < (int64_t)1 << 31 && Sk < (int64_t)1 << 31, "attn_fwd: too large");
  if (int rc = check_bhsd("attn_fwd", "q", q, q_strides, D)) return rc;
  if (int rc = check_bhsd("attn_fwd", "k", k, k_strides, D)) return rc;
  if (int rc = check_bhsd("attn_fwd", "v", v, v_strides, D)) return rc;
  TB_CHECK(o != nullptr && aligned16(o) && (o16 == nullptr || aligned16(o16)), "attn_fwd: bad output");
  if (bias) TB_CHECK(bias_strides != nullptr, "attn_fwd: bias strides missing");
  TB_CHECK(dropout_p >= 0.f && dropout_p < 1.f, "attn_fwd: dropout_p must be in [0, 1)");
  const WsLayout w = fwd_ws(B, H, Hkv, Sq, Sk, D);
  TB_CHECK(ws != nullptr && ws_bytes >= (int64_t)w.total, "attn_fwd: workspace too small");
  if (B == 0 || Sq == 0) return 0;
  TB_CHECK(Sk > 0, "attn_fwd: empty key sequence");
  hipStream_t st = as_stream(stream);
  float* pq = reinterpret_cast<float*>(ws);
  float* pk = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + w.off_k);
  float* pv = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + w.off_v);
  // S^T = K Q^T on k's and q's own bf16 rows where the head dim is a whole
  // staging width and there are no bias rows or dropout (TBF16_ATTN_KF16 forces
  // the fp16 k16 copy, for benchmarking); then q's and k's maxima are needed
  // only for the exponents the caller asks for
  const bool kbf = D == w.DP && w.DP <= 128 && !bias && dropout_p == 0.f && k_strides[2] < ((int64_t)1 << 23) &&
                   getenv("TBF16_ATTN_KF16") == nullptr;
  const bool derive_a = !kbf || exps != nullptr;
  {
    // partial per-head maxima of q, k and v (or of v alone) in one launch
    AmaxSegs segs;
    segs.n = derive_a ? 3 : 1;
    const AmaxSeg sv{(const uint16_t*)v, B * Hkv, Hkv, Sk, v_strides[0], v_strides[1], v_strides[2],
                     cdiv(Sk, w.nch_v), w.nch_v, pv};
    if (derive_a) {
      segs.seg[0] = AmaxSeg{(const uint16_t*)q, B * H, H, Sq, q_strides[0], q_strides[1], q_strides[2],
                            cdiv(Sq, w.nch_q), w.nch_q, pq};
      segs.seg[1] = AmaxSeg{(const uint16_t*)k, B * Hkv, Hkv, Sk, k_strides[0], k_strides[1], k_strides[2],
                            cdiv(Sk, w.nch_k), w.nch_k, pk};
      segs.seg[2] = sv;
    } else {
      segs.seg[0] = sv;
    }
    if (int rc = launch_head_amax3(segs, D, st)) return rc;
  }
  FwdParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.bias = (const uint16_t*)bias;
  p.bias_sb = bias ? bias_strides[0] : 0;
  p.bias_sh = bias ? bias_strides[1] : 0;
  p.bias_sq = bias ? bias_strides[2] : 0;
  p.B = (int)B; p.H = (int)H; p.Hkv = (int)Hkv; p.Sq = (int)Sq; p.Sk = (int)Sk; p.D = (int)D;
  p.scale_log2 = scale * kLog2e;
  p.v_exp = v_exp;
  p.part_q = pq; p.part_k = pk; p.part_v = pv;
  p.nch_q = (int)w.nch_q; p.nch_k = (int)w.nch_k; p.nch_v = (int)w.nch_v;
  p.o = (uint16_t*)o;
  p.lse = lse;
  p.o16 = (uint16_t*)o16;
  p.exps = exps;
  p.pair = 0;
  p.conv_k = !kbf;
  p.derive_a = derive_a;
  set_dropout(dropout_p, seed, p.drop_lo, p.drop_hi, p.drop_thr, p.drop_scale);
  char* wsb = reinterpret_cast<char*>(ws);
  p.ex = reinterpret_cast<int32_t*>(wsb + w.off_ex);
  p.k16 = reinterpret_cast<uint16_t*>(wsb + w.off_k16);
  p.vt16 = reinterpret_cast<uint16_t*>(wsb + w.off_vt16);
  p.Skp = (int)w.Skp;
  p.DPc = (int)w.DP;
  {
    const dim3 g((unsigned)(w.Skp / BKV), (unsigned)(B * Hkv));
    if (w.DP == 64) kv_prep_kernel<64><<<g, 256, 0, st>>>(p);
    else if (w.DP == 128) kv_prep_kernel<128><<<g, 256, 0, st>>>(p);
    else kv_prep_kernel<256><<<g, 256, 0, st>>>(p);
    TB_LAUNCH_CHECK("attn_fwd/kv_prep");
  }
  const char* ov = getenv("TBF16_ATTN_WAVES");  // benchmarking override: 4 or 8
  const int nw = ov ? atoi(ov) : 0;
  if (D <= 64) return launch_fwd_dp<64>(p, causal != 0, bias != nullptr, st, nw);
  if (D <= 128) return launch_fwd_dp<128>(p, causal != 0, bias != nullptr, st, nw);
  return launch_fwd_dp<256>(p, causal != 0, bias != nullptr, st, nw);
}
