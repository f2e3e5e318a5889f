/* tbf16_hip.h -- C ABI of the MI355X (gfx950) scaled-fp16 hot path.
 *
 * Drop-in boundary for tech-cosmos/turing-bf16's native extensions: every entry
 * point below replaces one pybind11 export of tbf16/csrc/{gemm_sm75,small_kernels}.cu (or a third-party
 * kernel the reference calls through torch), with the same argument meaning.
 * Reference citations are paths relative to the reference tree.
 *
 * Conventions
 *  - All tensor arguments are device pointers; shapes, strides (in elements) and
 *    the HIP stream (hipStream_t passed as void*) are plain integers/pointers.
 *  - The caller allocates every output and workspace; the library allocates
 *    nothing. Launches are asynchronous on `stream`; nothing synchronizes.
 *  - Return 0 on success, a negative TBF16_E* code on failure; the message is in
 *    tbf16_last_error() (thread-local). Preconditions are checked on the host
 *    before any launch, with the reference's messages where it has one.
 *  - Scale exponents are exchanged as int32 p (scale = 2^p); inverse scales as
 *    fp32 (2^-p), which is what the reference's Python API returns.
 */
#ifndef TBF16_HIP_H
#define TBF16_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TBF16_ABI_VERSION 3

#define TBF16_OK 0
#define TBF16_EINVAL (-1) /* bad shape, stride, alignment or dtype */
#define TBF16_ELAUNCH (-2) /* a HIP launch failed */
#define TBF16_EWS (-3)    /* workspace too small */

#define TBF16_DT_BF16 0
#define TBF16_DT_F16 1

/* Library identity. */
int tbf16_abi_version(void);
const char* tbf16_last_error(void);

/* Per-row scale exponents p[r] (scale 2^p puts max|x[r,:]|, or the L1 norm with
 * l1 != 0, in [2^(t-1), 2^t)); optional fp32 inverse scales 2^-p.
 * Replaces row_scale (tbf16/csrc/gemm_sm75.cu:243-253, kernel :27-47). x bf16
 * (M, K) row stride ldx; K % 8 == 0, ldx % 8 == 0, 16-byte aligned. */
int tbf16_row_exps(const void* x, int64_t M, int64_t K, int64_t ldx, int t, int l1, int32_t* exps,
                   float* s_inv, void* stream);

/* y16 = fp16(x * 2^p[r]) and s_inv[r] = 2^-p[r].
 * Replaces quantize_rows (tbf16/csrc/small_kernels.cu:275-287, kernel :35-74;
 * Python tbf16/ops.py:74-89). */
int tbf16_quantize_rows(const void* x, int64_t R, int64_t K, int64_t ldx, int t, int l1, void* y16, int64_t ldy,
                        float* s_inv, void* stream);

/* quantize_rows with the fp16 result written transposed: yT (K, R), row stride
 * ldyT >= R. Same exponents as tbf16_quantize_rows with l1 = 0. exps_ws: int32
 * (R,) workspace. Serves ScaledLinearFn.forward's saved x16 (tbf16/autograd.py:
 * 62-65) in the layout dW consumes. */
int tbf16_quantize_rows_t(const void* x, int64_t R, int64_t K, int64_t ldx, int t, void* yT, int64_t ldyT,
                          float* s_inv, int32_t* exps_ws, void* stream);

/* Column quantisation: amax[c] = max_r |x[r,c] * row_mul[r]|, y = fp16((x * row_mul)
 * * 2^p[c]), s_inv[c] = 2^-p[c]; row_mul (R,) fp32 powers of two or NULL. The fp16
 * result is written transposed: yT (K, R), row stride ldyT >= R.
 * Replaces quantize_cols (tbf16/csrc/small_kernels.cu:318-340, kernels :136-184;
 * Python tbf16/autograd.py:26-36). ws: tbf16_quantize_cols_ws_bytes(R, K) bytes. */
size_t tbf16_quantize_cols_ws_bytes(int64_t R, int64_t K);
int tbf16_quantize_cols_t(const void* x, int64_t R, int64_t K, int64_t ldx, int t, const float* row_mul, void* yT,
                          int64_t ldyT, float* s_inv, void* ws, int64_t ws_bytes, void* stream);

/* Fused scaled linear: y = bf16((sum_k fp16(x[m,k] * 2^p[m]) * w16[n,k]) * 2^-p[m]
 * * ws[n] + bias[n]), fp16 MFMA with fp32 accumulation, p from tbf16_row_exps(x, t,
 * l1) computed inside this call. One bf16 rounding.
 * x bf16 (M, K); w16 fp16 (N, K); ws fp32 (N,); bias bf16 (N,) or NULL; y bf16
 * (M, N). cfg < 0 picks the tile shape. workspace: tbf16_linear_ws_bytes(M, K, N,
 * cfg) bytes, 16-byte aligned; its first M int32 receive the row exponents p.
 * With the decode configurations, and with tiles of at most 128 columns at K >=
 * 1024, x is quantised once, as the reference's small-M path does: the row
 * inverse scales and x's scaled fp16 copy go into the workspace too, and the
 * GEMM runs on fp16 operands (the same output as converting x inside it). Where
 * the tiles would leave half of the CUs idle (K >= 2048, at most 8 MiB of partial
 * sums), K is split in two: fp32 partial sums go into the workspace and a second
 * kernel adds them in a fixed order and applies the epilogue. Replaces linear (tbf16/csrc/gemm_sm75.cu:257-284) and, at
 * 2 <= M < 256, quantize_rows + cuBLAS + epilogue (tbf16/ops.py:163-178) without
 * its fp16 intermediate. */
size_t tbf16_linear_ws_bytes(int64_t M, int64_t K, int64_t N, int cfg);
int tbf16_linear(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w16, int64_t N, int64_t ldw,
                 const float* ws, const void* bias, void* y, int64_t ldy, int t, int l1, int cfg, void* workspace,
                 void* stream);

/* tbf16_linear without a workspace argument and without allocating anything: the
 * workspace lives in a static device array of TBF16_NOALLOC_SCRATCH_BYTES per GPU
 * (12 MiB, held until the process ends). No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). Where x's fp16 copy does not fit in the array,
 * a tile configuration converts x inside the GEMM instead (the same output); M
 * above TBF16_NOALLOC_MAX_ROWS, or a decode-sized call (M <= 128) whose copy does
 * not fit (K beyond ~48k at M = 128), is rejected (TBF16_EINVAL). The array used is
 * the current device's, so the stream must belong to the current device (a stream
 * of another device is rejected). Calls that overlap on one GPU (concurrent streams
 * or threads) share the array and race. Same arguments and results as tbf16_linear
 * otherwise. */
#define TBF16_NOALLOC_MAX_ROWS (1 << 20)
#define TBF16_NOALLOC_SCRATCH_BYTES (12 << 20)
int tbf16_linear_noalloc(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w16, int64_t N, int64_t ldw,
                         const float* ws, const void* bias, void* y, int64_t ldy, int t, int l1, int cfg,
                         void* stream);

/* tbf16_linear with the row exponents already computed (exps int32 (M,), e.g. by
 * tbf16_quantize_rows_t): the training forward, which quantises x once for the
 * saved fp16 copy and for the GEMM (tbf16/autograd.py:60-68). */
int tbf16_linear_exps(const void* x, int64_t M, int64_t K, int64_t ldx, const int32_t* exps, const void* w16,
                      int64_t N, int64_t ldw, const float* ws, const void* bias, void* y, int64_t ldy, int cfg,
                      void* stream);

/* GEMM on already-quantised fp16 operands, both K-contiguous:
 * y = bf16((a16 @ b16^T) * sa[m] * sb[n] + bias[n]) with fp32 accumulation.
 * Replaces the cuBLAS fp16 GEMM + epilogue pair of linear_q (tbf16/ops.py:167-178,
 * small_kernels.cu:289-302) and _scaled_mm (tbf16/autograd.py:49-55). */
int tbf16_gemm_f16(const void* a16, int64_t M, int64_t K, int64_t lda, const float* sa, const void* b16, int64_t N,
                   int64_t ldb, const float* sb, const void* bias, void* y, int64_t ldy, int cfg, void* stream);

/* M = 1: y[n] = bf16((sum_k x[k] * w16[n,k]) * ws[n] + bias[n]) in fp32.
 * Replaces gemv (tbf16/csrc/small_kernels.cu:304-315, kernel :107-132). */
int tbf16_gemv(const void* x, const void* w16, int64_t N, int64_t K, int64_t ldw, const float* ws, const void* bias,
               void* y, void* stream);

/* Per-(b, h) max |x| over (S, D) into out fp32 (B, H). x (B, H, S, D) bf16 or fp16
 * with element strides (sb, sh, ss), contiguous D % 8 == 0.
 * Replaces head_amax (tbf16/csrc/small_kernels.cu:342-359, kernel :222-243). */
int tbf16_head_amax(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb, int64_t sh,
                    int64_t ss, float* out, void* stream);

/* y (contiguous B, H, S, D) = cast(x * 2^e[b, h]); e int32 with element strides
 * (e_sb, e_sh) so that broadcast exponents need no copy.
 * Replaces head_scale_cast (tbf16/csrc/small_kernels.cu:361-379, kernel :246-263). */
int tbf16_head_scale_cast(const void* x, int in_dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                          int64_t sh, int64_t ss, const int32_t* e, int64_t e_sb, int64_t e_sh, void* y,
                          int out_dtype, void* stream);

/* Scaled convolution input: per-sample exponents and the scaled fp16 copy.
 * x bf16 holds B samples of n elements each, back to back (a contiguous NC...
 * or channels-last tensor), 16-byte aligned; x16 fp16 has the same layout.
 * exps[b] = frexp(max |x[b]|) - t (1 - t for an all-zero or NaN sample, -t for
 * an infinite one); x16 = fp16(x * 2^-exps[b]) from fp32, one RNE rounding.
 * ws: tbf16_conv_input_ws_bytes(B, n) bytes of scratch.
 * Replaces the input half of _scaled_conv_forward (tbf16/conv.py:49-54:
 * vector_norm, frexp, ldexp, mul). */
size_t tbf16_conv_input_ws_bytes(int64_t B, int64_t n);
int tbf16_conv_input(const void* x, int64_t B, int64_t n, int t, int32_t* exps, void* x16, void* ws,
                     int64_t ws_bytes, void* stream);

/* Scaled convolution epilogue: out = bf16(y16 * (2^exps[b] * ws[o]) + bias[o]),
 * the scale an fp32 product, the sum rounded to fp32 then to bf16. y16 fp16 and
 * out bf16 are (B, O, P) contiguous (channels_last = 0) or (B, P, O)
 * (channels_last = 1), P = prod(output spatial), 16-byte aligned; ws fp32 (O,)
 * inverse weight scales; bias fp32 (O,) or NULL.
 * Replaces the output half of _scaled_conv_forward (tbf16/conv.py:56-60:
 * ldexp, mul / addcmul). */
int tbf16_conv_epilogue(const void* y16, int64_t B, int64_t O, int64_t P, int channels_last, const int32_t* exps,
                        const float* ws, const float* bias, void* out, void* stream);

/* Scaled attention forward (flash-style, no S x S buffer).
 * Exponents (tbf16/attention.py:38-48): eq/ek = max over heads of frexp(amax),
 * a = clamp(floor((ek - eq) / 2)), ev[b, hkv] = frexp(amax v[b, hkv]) - v_exp.
 * Computes softmax((q 2^a)(k 2^-a)^T * scale + bias) (v 2^-ev) on fp16 MFMA with
 * fp32 online softmax and writes o = bf16(O / l * 2^ev) once.
 * q (B, H, Sq, D), k/v (B, Hkv, Sk, D) bf16, strides in elements (b, h, s) with
 * contiguous D; D % 8 == 0, D <= 256; H % Hkv == 0. bias: optional fp16 additive
 * mask read at bias[b*bsb + h*bsh + i*bsq + j] (strides may be 0 to broadcast).
 * causal: key j visible to query i iff j <= i (top-left, as torch).
 * Outputs: o bf16 (B, H, Sq, D) contiguous; optional lse fp32 (B, H, Sq) in log2
 * units of (logit * scale * log2(e)); optional o16 fp16 (B, H, Sq, D) = O / l
 * (saved for the backward); optional exps int32 [2 + B*Hkv] = {a, 0, ev...}.
 * dropout_p in [0, 1): attention weights dropped by a counter-based hash of
 * (seed, b*H + h, query, key) (MurmurHash3 fmix32 finalizer, see the device
 * helpers), kept ones scaled by 1 / (1 - p); l and lse use the undropped weights,
 * so tbf16_attn_bwd with the same seed and p regenerates the mask. The reference
 * passes dropout_p to torch's kernel, whose Philox stream differs: masks are not
 * comparable bit for bit.
 * Replaces prepare_qkv + torch's fp16 memory-efficient SDPA + head_scale
 * (tbf16/attention.py:56-65) and _eff_fwd (tbf16/autograd.py:155-164). */
size_t tbf16_attn_fwd_ws_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D);
int tbf16_attn_fwd(const void* q, const void* k, const void* v, int64_t B, int64_t H, int64_t Hkv, int64_t Sq,
                   int64_t Sk, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const void* bias, const int64_t* bias_strides, float scale, int causal,
                   int v_exp, float dropout_p, uint64_t seed, void* o, float* lse, void* o16, int32_t* exps,
                   void* ws, int64_t ws_bytes, void* stream);

/* Scaled attention backward for one value of the dO target exponent t_do.
 * e = max(frexp(amax dout[b,h]) + ev_q[b,h]), G = t_do - e, dO16 = fp16(dout *
 * 2^(ev_q + G)). dq = bf16(scale * dS K16 * 2^(a-G)), dk = bf16(scale * sum_grp
 * dS^T Q16 * 2^(-a-G)), dv = bf16(sum_grp P^T dO16 * 2^(-ev-G)), all from fp32.
 * *overflow (device int32) receives the bit pattern of the largest magnitude of
 * the gradients in the scaled fp16 domain (dq16, dk16, dv16 of every query head,
 * taken before a GQA group is summed, as the reference checks them; +inf if any
 * is not finite); at 65520 and above (bits >= 0x477FF000) they would overflow
 * fp16, the reference's retry condition (tbf16/autograd.py:177-189). exps_out
 * int32 [2] = {e, G}. gate: null, or the overflow word of an earlier call with the
 * same arguments and workspace. A gated call is the reference's retry loop run on
 * the device: when that call's maximum was below 65520 it leaves the outputs as
 * they are and copies the gate's word into its own; else it runs at t_do - 8 r
 * with r the number of retries the reference would take (each retry scales every
 * value by 2^-8, at most 5), writing the same outputs and its own overflow word;
 * no host round trip is needed between the two calls. With GQA (H > Hkv) the
 * workspace also holds each query head's fp32 dK and dV, summed over the group in
 * head order (the reference's fp32 _reduce_kv). Inputs are the forward's q, k,
 * v, o16, lse and exps; same shape
 * rules as the forward (D % 8 == 0, D <= 256); dropout_p and seed as given to
 * the forward (its mask is regenerated: dV from P o Z, dS = P o (Z o dP - delta)
 * with Z = keep / (1 - p)).
 * Replaces torch's _scaled_dot_product_efficient_attention_backward call and the
 * surrounding scaling (tbf16/autograd.py:166-193). */
size_t tbf16_attn_bwd_ws_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D);
int tbf16_attn_bwd(const void* q, const void* k, const void* v, const void* o16, const float* lse,
                   const void* dout, const int32_t* exps_fwd, int64_t B, int64_t H, int64_t Hkv, int64_t Sq,
                   int64_t Sk, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* do_strides, const void* bias,
                   const int64_t* bias_strides, float scale, int causal, int t_do, float dropout_p, uint64_t seed,
                   void* dq, void* dk, void* dv, int32_t* exps_out, int32_t* overflow, const int32_t* gate,
                   void* ws, int64_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TBF16_HIP_H */
