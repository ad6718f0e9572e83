/* C ABI of libttt_amd.so: the TTT-Linear / TTT-MLP mini-batch inner loop on
 * MI355X (gfx950), forward, backward and the MLP fixed-weight readout.
 *
 * Conventions shared by every entry point
 *   - Every pointer is device memory, contiguous, row-major, with the layouts
 *     given per argument.  B batch, H heads, NC mini-batches, K tokens per
 *     mini-batch, F head dim, FF MLP hidden width, G checkpoint group size
 *     (1..NC), NK = ceil(NC / G).  K, F and FF are multiples of 16 with
 *     K <= 64, F <= 256, FF <= 1024.  K = 16 with F in {32, 64} (and, for the
 *     MLP, FF in {64, 128, 256}) runs the specialised kernels; every other
 *     shape runs the general-shape kernels, whose forward also needs the
 *     `saved` buffer (it holds the state entering every mini-batch and the
 *     per-mini-batch scratch; the backward reads it).  The fixed-weight
 *     kernels (cached readout, memo combiner) take any K, F in {32, 64} and
 *     FF in {32, 64, 128, 256}.
 *   - Activations (XQ, XK, XV, out and their gradients) share one dtype,
 *     `dtype` (TTT_DTYPE_F32, TTT_DTYPE_BF16 or TTT_DTYPE_F16; both 16-bit
 *     types are read into the matrix cores as they are and accumulate in fp32).  Fast-weight state, LayerNorm
 *     parameters, checkpoints, memo snapshots and weight gradients are fp32.
 *   - eta comes in one of two forms, chosen by `eta_rule` (enum ttt_eta_rule):
 *     TTT_ETA_DENSE: `eta` is the full [B,H,NC,K,K] tensor in the activation
 *     dtype, as ops/ttt_linear.py and ops/ttt_mlp.py take it, and the
 *     backward writes the dense [B,H,NC,K,K] gradient into `deta`;
 *     TTT_ETA_DENSE_F32: the same dense eta and gradient in fp32 whatever
 *     `dtype` is (the reference's kernels take eta in its own dtype; a 16-bit
 *     deta overflows fp16 where the inputs are not normalised);
 *     TTT_ETA_LAYER / TTT_ETA_CAUSAL: `eta` is the per-token learning rate
 *     lr [B,H,NC,K] fp32 (TTTBase.get_eta, ttt_layer.py:151-163) that the
 *     kernels expand on chip (LAYER: eta[i][j] = lr[j]/K for every row i, the
 *     layer's own rule, ttt_layer.py:309; CAUSAL: eta[i][j] = lr[j]/(i+1) for
 *     j <= i, else 0), and the backward writes dlr [B,H,NC,K] fp32
 *     (dlr[j] = sum_i deta[i][j] * d eta[i][j] / d lr[j]) into `deta`.
 *   - The caller allocates every buffer; nothing is allocated or kept between
 *     calls.  `stream` is a hipStream_t (NULL = the null stream); launches are
 *     asynchronous on it.
 *   - Arguments are validated on the host before any launch.  Return value:
 *     TTT_OK or a negative TTT_ERR_* code (see ttt_error_string).
 *   - Semantics are those of the reference's PyTorch ops path: dual form with
 *     a general KxK eta (no implicit tril), LayerNorm eps given by `eps`
 *     (the ops path uses 1e-8), dense KxK eta gradient.
 */
#ifndef TTT_AMD_H_
#define TTT_AMD_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTT_AMD_ABI_VERSION 11

enum ttt_dtype { TTT_DTYPE_F32 = 0, TTT_DTYPE_BF16 = 1, TTT_DTYPE_F16 = 2 };

enum ttt_eta_rule { TTT_ETA_DENSE = 0, TTT_ETA_LAYER = 1, TTT_ETA_CAUSAL = 2, TTT_ETA_DENSE_F32 = 3 };

enum ttt_status {
  TTT_OK = 0,
  TTT_ERR_SHAPE = -1,     /* unsupported or inconsistent shape */
  TTT_ERR_DTYPE = -2,     /* unsupported dtype */
  TTT_ERR_NULL = -3,      /* required pointer is NULL */
  TTT_ERR_ALIGN = -4,     /* pointer not 16-byte aligned */
  TTT_ERR_HIP = -5,       /* launch failed (hipGetLastError) */
  TTT_ERR_WORKSPACE = -6, /* workspace missing or too small */
  TTT_ERR_ARG = -7,       /* other invalid argument (eps, G, M, eta_rule, option) */
  TTT_ERR_TIMEOUT = -8,   /* ttt_mlp_bwd_check: a dXQ/dXK worker gave up waiting */
  TTT_ERR_SCRATCH = -9    /* ttt_mlp_bwd_noalloc: problem larger than its static scratch */
};

/* ABI version of the loaded library (TTT_AMD_ABI_VERSION). */
int ttt_abi_version(void);

/* Static description of a status code. */
const char* ttt_error_string(int status);

/* TTT-Linear forward over all NC mini-batches of B*H chains.
 * Replaces ttt_linear_scan_forward (kernels/linear_forward.py:5-148) as
 * launched by TritonLinear._forward_core (linear_triton.py:62-144), and is
 * the forward of ops.ttt_linear (ops/ttt_linear.py:57-84).
 *   XQ, XK, XV  [B,H,NC,K,F] dtype      eta [B,H,NC,K,K] dtype, or lr [B,H,NC,K] fp32 (eta_rule)
 *   ln_w, ln_b  [H,F] fp32              W1_init [B,H,F,F], b1_init [B,H,1,F] fp32
 *   out         [B,H,NC,K,F] dtype      (XQ + LN(Z1_bar) per mini-batch)
 *   W1_last, b1_last  [B,H,F,F], [B,H,1,F] fp32, final state (both or neither)
 *   W1_ckpt, b1_ckpt  [B,H,NK,F,F], [B,H,NK,1,F] fp32, state entering
 *                     mini-batch k*G (both or neither; needed by the backward)
 *   saved             NULL, or >= ttt_linear_saved_bytes(...) bytes: receives,
 *                     for every mini-batch, the inner-loss gradient and the
 *                     normalised pre-LN values with their statistics that
 *                     ttt_linear_bwd needs.  It has no counterpart in the
 *                     reference, whose backward re-runs each checkpoint group
 *                     forward to recover them.
 * NC times the per-mini-batch saved size must stay below 2^31 bytes. */
int ttt_linear_fwd(const void* XQ, const void* XK, const void* XV, const void* eta,
                   const float* ln_w, const float* ln_b, const float* W1_init, const float* b1_init,
                   int B, int H, int NC, int K, int F, int G, int dtype, int eta_rule, float eps,
                   void* out, float* W1_last, float* b1_last, float* W1_ckpt, float* b1_ckpt,
                   void* saved, size_t saved_bytes, void* stream);

/* Bytes of the saved buffer of ttt_linear_fwd / ttt_linear_bwd: with the
 * specialised kernels B*H*NC mini-batches x (3 * F * 64 + 256); with the
 * general-shape kernels, per chain, the state entering every mini-batch and
 * the fp32 scratch of one mini-batch; 0 for unsupported sizes. */
size_t ttt_linear_saved_bytes(int B, int H, int NC, int K, int F);

/* TTT-Linear backward: gradients of sum(out * dout) wrt every input, the
 * final state's gradient taken as zero (the ops path discards W_last).
 * Replaces ttt_linear_scan_backward (kernels/linear_backward.py:207-520) as
 * launched by TritonLinear._backward_core (linear_triton.py:146-265).
 *   W1_ckpt           weight checkpoints written by ttt_linear_fwd with the same G
 *   W1_last           the final weight written by that ttt_linear_fwd call
 *   dout              [B,H,NC,K,F] dtype
 *   dXQ, dXK, dXV     [B,H,NC,K,F] dtype;  deta [B,H,NC,K,K] dtype (dense), or
 *                     dlr [B,H,NC,K] fp32 (eta_rule LAYER / CAUSAL)
 *   dW1, db1          [B,H,F,F], [B,H,1,F] fp32 (gradient wrt W1_init, b1_init)
 *   dln_w, dln_b      [B,H,F] fp32 per-chain partials; sum over B for [H,F]
 *   saved             the saved buffer written by that ttt_linear_fwd call
 *                     (saved_bytes >= ttt_linear_saved_bytes(...))
 * The bias checkpoints are not needed: the saved values carry everything the
 * bias entered. */
int ttt_linear_bwd(const void* XQ, const void* XK, const void* XV, const void* eta,
                   const float* ln_w, const float* ln_b, const float* W1_ckpt, const float* W1_last,
                   const void* dout, int B, int H, int NC, int K, int F, int G, int dtype, int eta_rule, float eps,
                   void* dXQ, void* dXK, void* dXV, void* deta, float* dW1, float* db1,
                   float* dln_w, float* dln_b, const void* saved, size_t saved_bytes, void* stream);

/* TTT-MLP forward (2-layer GELU(tanh) fast-weight MLP) over all NC
 * mini-batches.  Replaces ttt_mlp_scan_forward (kernels/mlp_forward.py:6-237)
 * as launched by TritonMLP._forward_core (mlp_triton.py:71-197), and is the
 * forward of ops.ttt_mlp (ops/ttt_mlp.py:70-99).
 *   W1_init [B,H,F,FF], b1_init [B,H,1,FF], W2_init [B,H,FF,F], b2_init [B,H,1,F] fp32
 *   out               [B,H,NC,K,F] dtype
 *   *_last            final state, shapes of *_init (all four or none)
 *   *_ckpt            [B,H,NK,...] state entering mini-batch k*G: W1_ckpt, or
 *                     none; b1_ckpt, W2_ckpt and b2_ckpt are each optional (the
 *                     backward reads W1's only)
 *   *_memo            [B,H,NS,...], NS = ceil(NC/M): state after mini-batch
 *                     s*M has been applied (all four or none; M >= 1 then;
 *                     M > NC gives NS = 1, as the reference's memo loop does)
 *   saved             NULL, or >= ttt_mlp_saved_bytes(...) bytes: receives, for
 *                     every mini-batch, the state-update operands and the
 *                     activations ttt_mlp_bwd needs.  It has no counterpart in
 *                     the reference, whose backward re-runs each checkpoint
 *                     group forward to recover them.
 * Per-chain slabs are addressed with 32-bit offsets: NC * F * FF * 4 and NC
 * times the per-mini-batch saved size must stay below 2^31 bytes. */
int ttt_mlp_fwd(const void* XQ, const void* XK, const void* XV, const void* eta,
                const float* ln_w, const float* ln_b, const float* W1_init, const float* b1_init,
                const float* W2_init, const float* b2_init,
                int B, int H, int NC, int K, int F, int FF, int G, int M, int dtype, int eta_rule, float eps,
                void* out, float* W1_last, float* b1_last, float* W2_last, float* b2_last,
                float* W1_ckpt, float* b1_ckpt, float* W2_ckpt, float* b2_ckpt,
                float* W1_memo, float* b1_memo, float* W2_memo, float* b2_memo,
                void* saved, size_t saved_bytes, void* stream);

/* Bytes of the saved buffer of ttt_mlp_fwd / ttt_mlp_bwd: with the
 * specialised kernels B*H*NC mini-batches x ((7 FF + F) * K * sizeof(dtype)
 * + (FF + F) * 4 + 3 * F * 64 + 4096); with the general-shape kernels, per
 * chain, the state entering every mini-batch and the fp32 scratch of one
 * mini-batch. */
size_t ttt_mlp_saved_bytes(int B, int H, int NC, int K, int F, int FF, int dtype);

/* Bytes of device workspace ttt_mlp_bwd uses: B*H*NC mini-batches x
 * (2 * FF * K * sizeof(dtype) + 2 * F * 64), then (4 + B*H*NC) 4-byte control
 * words rounded up to 256 bytes (specialised kernels; all of it required);
 * with F = FF = 32 and K <= 64 (the register-resident kernels) B*H*NC x
 * 48 KB at K = 64 (less at smaller K), the handoff of their two-launch form,
 * which they use when given that much and otherwise run in one launch with
 * at least 256 bytes; 256 with the other general shapes, which keep their
 * scratch in `saved`. */
size_t ttt_mlp_bwd_workspace_bytes(int B, int H, int NC, int K, int F, int FF, int dtype);

/* TTT-MLP backward: gradients of sum(out * dout) wrt every input (final
 * state's gradient zero, as in the ops path).  Replaces ttt_mlp_scan_backward
 * (kernels/mlp_backward.py:247-651) as launched by TritonMLP._backward_core
 * (mlp_triton.py:200-351).
 *   W1_ckpt          weight checkpoints written by ttt_mlp_fwd with the same G
 *                    (b1_ckpt, W2_ckpt, b2_ckpt are not read and may be NULL)
 *   *_last           the final state written by that ttt_mlp_fwd call
 *   dout             [B,H,NC,K,F] dtype
 *   dXQ, dXK, dXV    [B,H,NC,K,F] dtype;  deta [B,H,NC,K,K] dtype (dense), or
 *                    dlr [B,H,NC,K] fp32 (eta_rule LAYER / CAUSAL)
 *   dW1, db1, dW2, db2  fp32, shapes of W1_init ... (gradient wrt the initial state)
 *   dln_w, dln_b     [B,H,F] fp32 per-chain partials; sum over B for [H,F]
 *   saved            the saved buffer written by that ttt_mlp_fwd call
 *                    (saved_bytes >= ttt_mlp_saved_bytes(...))
 *   workspace        scratch of ttt_mlp_bwd_workspace_bytes(...) bytes (at
 *                    least 256 outside the specialised kernels, above): dZ1b,
 *                    dZ1 and partial dXQ/dXK per mini-batch, handed from the
 *                    reverse sweep to the pass that forms dXQ/dXK, and that
 *                    pass's control words; or the register-resident
 *                    kernels' readout-path terms per mini-batch
 * When one chain's sweep fits per CU with CUs to spare (B*H + 16 <= CUs), the
 * dXQ/dXK pass runs in the sweep's launch on the spare CUs, each worker
 * waiting (bounded by TTT_OPT_MLP_BWD_POLL_LIMIT polls) for the checkpoint
 * group it takes.  A worker that gives up writes NaN into that group's dXQ
 * and dXK and raises a timeout word; ttt_mlp_bwd_check reads it.  Otherwise,
 * or with TTT_OPT_MLP_BWD_FUSED = 0, the pass is a second launch. */
int ttt_mlp_bwd(const void* XQ, const void* XK, const void* XV, const void* eta,
                const float* ln_w, const float* ln_b, const float* W1_ckpt, const float* b1_ckpt,
                const float* W2_ckpt, const float* b2_ckpt, const float* W1_last, const float* b1_last,
                const float* W2_last, const float* b2_last, const void* dout,
                int B, int H, int NC, int K, int F, int FF, int G, int dtype, int eta_rule, float eps,
                void* dXQ, void* dXK, void* dXV, void* deta, float* dW1, float* db1, float* dW2, float* db2,
                float* dln_w, float* dln_b, const void* saved, size_t saved_bytes, void* workspace,
                size_t workspace_bytes, void* stream);

/* Fixed-weight TTT-MLP readout over a segment of NS mini-batches:
 *   out = XQ + LN_eps(gelu(XQ W1 + b1) W2 + b2)   (no state update)
 * with the weights of each (b,h) chain.  Replaces mlp_cached_readout_triton
 * (kernels/mlp_cached_readout.py:112-143) and its kernel (:7-109), as called
 * per cached memo slice from ttt_layer.py:542-552; the residual the
 * reference adds on the host (:143) is fused.  The reference uses eps 1e-6.
 *   XQ               [B,H,NS,K,F] dtype
 *   W1, b1, W2, b2   fp32; chain c = b*H + h reads W1 + c*S*F*FF,
 *                    b1 + c*S*FF, W2 + c*S*FF*F, b2 + c*S*F.  S = 1 for
 *                    [B,H,...] tensors; S = number of stacked states when the
 *                    pointers address slice j of [B,H,S,...] memo tensors,
 *                    so a memo slice is read in place.
 *   out              [B,H,NS,K,F] fp32 */
int ttt_mlp_cached_readout(const void* XQ, const float* W1, const float* b1, const float* W2,
                           const float* b2, const float* ln_w, const float* ln_b,
                           int B, int H, int NS, int K, int F, int FF, int S, int dtype, float eps,
                           float* out, void* stream);

/* Bytes of the gates buffer of ttt_mlp_memo_combine / _bwd: B*H chains x
 * (2*NS*NC*K + 2*NC*K + NS*F) floats (rounded up to 16 bytes), NS = ceil(NC/M);
 * 0 for unsupported sizes. */
size_t ttt_mlp_memo_gates_bytes(int B, int H, int NC, int K, int F, int M);

/* Bytes of the full workspace of ttt_mlp_memo_combine / _bwd: the gates
 * buffer and, for bf16, behind it (at the gates' size rounded up to 256
 * bytes) one LDS image per memo state (B*H*NS of them: the state's W1 and W2
 * as bf16 MFMA operand frags and its biases), which the forward call writes
 * once and both calls copy straight into LDS instead of converting every
 * state for every workgroup.  A gates buffer of at least this size takes
 * that path; one of at least ttt_mlp_memo_gates_bytes the converting one
 * (the same results).  0 for unsupported sizes.  No counterpart in the
 * reference. */
size_t ttt_mlp_memo_workspace_bytes(int B, int H, int NC, int K, int F, int FF, int M, int dtype);

/* TTT-MLP memory-cache combiner: the segment loop of TTTMLP.ttt
 * (ttt_layer.py:506-561, its cached-readout calls ttt_layer.py:542-552) in
 * three launches.  Segments of M mini-batches; for a token of segment i >= 1,
 * gamma = softmax over j = 0..i of XU . mean(XK over segment j), and
 *   out = gamma_i XQW + sum_{j<i} gamma_j (XQ + LN_eps(gelu(XQ W1_j + b1_j) W2_j + b2_j) ln_w + ln_b);
 * segment 0 keeps XQW.  Each (b,h) chain uses its own memo states.
 *   XQ, XK, XU, XQW   [B,H,NC,K,F] dtype      out [B,H,NC,K,F] dtype
 *   W1_memo ...       [B,H,NS,F,FF], [B,H,NS,1,FF], [B,H,NS,FF,F], [B,H,NS,1,F] fp32
 *                     (the memo output of ttt_mlp_fwd with the same M)
 *   ln_w, ln_b        [H,F] fp32;  eps: the cached readout's (1e-6 there)
 *   gates             >= ttt_mlp_memo_gates_bytes(...) bytes (better
 *                     ttt_mlp_memo_workspace_bytes(...)); receives the gates,
 *                     segment summaries and memo-state images, which
 *                     ttt_mlp_memo_combine_bwd reads
 * NS = ceil(NC/M) <= 256.  No counterpart in the reference's C-level code (it is
 * Python there); replaces the loop body, not a kernel. */
int ttt_mlp_memo_combine(const void* XQ, const void* XK, const void* XU, const void* XQW,
                         const float* W1_memo, const float* b1_memo, const float* W2_memo,
                         const float* b2_memo, const float* ln_w, const float* ln_b,
                         int B, int H, int NC, int K, int F, int FF, int M, int dtype, float eps,
                         void* out, float* gates, size_t gates_bytes, void* stream);

/* Backward of ttt_mlp_memo_combine: gradients wrt XK, XU and XQW.  As in
 * the reference, the cached readouts carry no gradient and a segment's
 * summary carries one only as the current summary of its own tokens' gates
 * (ttt_layer.py:519,528; it is cached detached, :521,559): dXK is the same
 * for every token of a segment, and 0 in segment 0.  `gates` and
 * `gates_bytes` as given to the forward call (its gradient part is
 * overwritten); dXK, dXU, dXQW
 * [B,H,NC,K,F] dtype. */
int ttt_mlp_memo_combine_bwd(const void* XQ, const void* XU, const void* XQW, const float* W1_memo,
                             const float* b1_memo, const float* W2_memo, const float* b2_memo,
                             const float* ln_w, const float* ln_b, const void* dout,
                             int B, int H, int NC, int K, int F, int FF, int M, int dtype, float eps,
                             float* gates, size_t gates_bytes, void* dXK, void* dXU, void* dXQW,
                             void* stream);

/* ---- the producer and consumer around the inner loop (ttt_layer.py) ----
 * Shapes: B batch, L = NC*K tokens, H heads, F head dim (32 or 64), K a
 * multiple of 16 up to 64, D = H*F <= 1024.  Activations in `dtype`, everything else fp32. */

/* Bytes of the per-block LayerNorm-parameter gradient partials of
 * ttt_qkvu_producer_bwd / ttt_post_norm_bwd: ceil(B*L/32) blocks x 2 x D
 * floats; the caller sums them over blocks (dln_w = sum[:, 0], dln_b =
 * sum[:, 1], each [D] = [H,F]).  0 for unsupported sizes. */
size_t ttt_layer_io_partial_bytes(int B, int L, int H, int F);

/* The layer's input preprocessing after its projections, written straight
 * into the inner loop's layouts.  Replaces, in TTTBase.process_input
 * (ttt_layer.py:261-309): the L2 normalisation of XQ, XK, XU (:279-281,
 * x / max(|x|, 1e-12)), RoPE at each token's position (:287-300 with
 * utils.py:97-123), ln_reconstruction_target (:227-243, :302; unbiased std,
 * `eps` = 1e-8 there), reshape_to_mini_batch (:245-259) and get_eta
 * (:151-163; lr = base_lr * sigmoid(logit) / F, before the layer's 1/K row
 * repeat, which the inner loop's TTT_ETA_LAYER rule applies on chip).
 *   proj     [B*L][ld] dtype: per token XQ | XK | XV | XU (D each, head-major)
 *            | H lr logits (ttt_lr_weight . x + ttt_lr_bias) | padding;
 *            ld >= 4*D + H, ld % 4 == 0 (one fused projection GEMM gives it)
 *   rope     [L][F/2][2] fp32: cos, sin of the angle of pair p at position t
 *   ln_w, ln_b  [H,F] fp32 (ttt_norm_weight / ttt_norm_bias)
 *   XQ, XK, XV, XU  [B,H,NC,K,F] dtype (XV = the reconstruction target)
 *   lr       [B,H,NC,K] fp32 */
int ttt_qkvu_producer_fwd(const void* proj, int ld, const float* rope, const float* ln_w, const float* ln_b,
                          int B, int L, int H, int K, int F, float base_lr, float eps, int dtype,
                          void* XQ, void* XK, void* XV, void* XU, float* lr, void* stream);

/* Backward of ttt_qkvu_producer_fwd (it recomputes the forward from proj):
 * given the gradients of its outputs (dlr may be NULL: no lr gradient),
 * writes the gradient of every proj row (padding columns zeroed) and the
 * LayerNorm-parameter partials of the reconstruction target. */
int ttt_qkvu_producer_bwd(const void* proj, int ld, const float* rope, const float* ln_w, const float* ln_b,
                          const void* dXQ, const void* dXK, const void* dXV, const void* dXU, const float* dlr,
                          int B, int L, int H, int K, int F, float base_lr, float eps, int dtype,
                          void* dproj, float* partial, size_t partial_bytes, void* stream);

/* The layer's output path before `wo`: the inner loop's output [B,H,NC,K,F]
 * permuted and reshaped to [B, L, D] (ttt_layer.py:406,420 / :563-564) and
 * LayerNorm-ed over D with gamma, beta [D] fp32 (post_norm, ttt_layer.py:78,349;
 * biased variance, `eps` 1e-6 there).  out [B,L,D] dtype; stats [B*L][2] fp32
 * (mean, 1/sigma) for the backward. */
int ttt_post_norm_fwd(const void* XQW, const float* gamma, const float* beta, int B, int L, int H, int K, int F,
                      float eps, int dtype, void* out, float* stats, void* stream);

/* Backward of ttt_post_norm_fwd: dXQW [B,H,NC,K,F] dtype and the gamma/beta
 * gradient partials. */
int ttt_post_norm_bwd(const void* XQW, const float* gamma, const float* stats, const void* dout,
                      int B, int L, int H, int K, int F, int dtype, void* dXQW, float* partial,
                      size_t partial_bytes, void* stream);

/* Bytes of the static device scratch of ttt_mlp_bwd_noalloc (per GPU). */
#define TTT_MLP_BWD_NOALLOC_SCRATCH_BYTES (64u << 20)

/* ttt_mlp_bwd with no workspace argument and no allocation of any kind: the
 * workspace (what ttt_mlp_bwd_workspace_bytes sizes) lives in a static device
 * array of TTT_MLP_BWD_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends.  No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Problems whose workspace exceeds the scratch return
 * TTT_ERR_SCRATCH (at F64 FF256 bf16 that is B*H*NC > 2730 mini-batch
 * slots, e.g. B1 H12 T2048 fits and B16 H12 T2048 does not).  All calls on one
 * GPU share its scratch, which keeps the last call's contents; the call clears
 * the words that must start at zero itself.  Calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the caller.
 * Arguments and results are ttt_mlp_bwd's. */
int ttt_mlp_bwd_noalloc(const void* XQ, const void* XK, const void* XV, const void* eta,
                        const float* ln_w, const float* ln_b, const float* W1_ckpt, const float* b1_ckpt,
                        const float* W2_ckpt, const float* b2_ckpt, const float* W1_last, const float* b1_last,
                        const float* W2_last, const float* b2_last, const void* dout,
                        int B, int H, int NC, int K, int F, int FF, int G, int dtype, int eta_rule, float eps,
                        void* dXQ, void* dXK, void* dXV, void* deta, float* dW1, float* db1, float* dW2,
                        float* db2, float* dln_w, float* dln_b, const void* saved, size_t saved_bytes,
                        void* stream);

/* Process-wide options of the library (no counterpart in the reference):
 *   TTT_OPT_MLP_BWD_POLL_LIMIT  polls of a checkpoint-group flag before a fused
 *                               dXQ/dXK worker of ttt_mlp_bwd gives up (>= 0;
 *                               default 4194304, about a second)
 *   TTT_OPT_MLP_BWD_FUSED       1 (default): the dXQ/dXK pass runs inside the
 *                               sweep's launch when it fits; 0: always a second
 *                               launch (no waits at all)
 *   TTT_OPT_SMALL_KERNELS       1 (default): shapes outside the specialised set
 *                               with F = 32 (FF = 32), K <= 64 run the
 *                               register-resident one-wave-per-chain kernels;
 *                               0: the staged general-shape kernels (same
 *                               interface and saved buffer)
 * ttt_set_option returns TTT_OK or TTT_ERR_ARG; ttt_get_option returns the
 * value, or -1 for an unknown option. */
enum ttt_option { TTT_OPT_MLP_BWD_POLL_LIMIT = 1, TTT_OPT_MLP_BWD_FUSED = 2, TTT_OPT_SMALL_KERNELS = 3 };
int ttt_set_option(int option, long long value);
long long ttt_get_option(int option);

/* Status of the last ttt_mlp_bwd call that used `workspace` (same sizes):
 * waits for `stream`, then returns TTT_OK, or TTT_ERR_TIMEOUT if a fused
 * dXQ/dXK worker gave up waiting for its checkpoint group (that group's dXQ
 * and dXK rows then hold NaN).  With workspace NULL (workspace_bytes is then
 * ignored) it reads the static scratch of ttt_mlp_bwd_noalloc on the current
 * device instead: the status of the last no-allocation call there.  Shapes
 * outside the specialised kernels have no fused workers: TTT_OK at once.  No
 * counterpart in the reference, whose backward has no cross-workgroup waits. */
int ttt_mlp_bwd_check(const void* workspace, size_t workspace_bytes, int B, int H, int NC, int K, int F,
                      int FF, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TTT_AMD_H_ */
