// Kernel-side parameter blocks and launchers (internal to libttt_amd.so).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/ttt_amd.h"
#include "ttt_tile.h"

namespace ttt {

struct LinearFwdParams {
  const void *XQ, *XK, *XV, *eta;
  const float *ln_w, *ln_b, *W_init, *b_init;
  void* out;
  float *W_last, *b_last, *W_ckpt, *b_ckpt;
  void* saved;  // per mini-batch values for the backward, LinSavedSlot layout (may be null)
  int B, H, NC, F, G, NK;
  int eta_rule;  // TTT_ETA_*: eta dense [NC][K][K] (activation type) or lr [NC][K] fp32
  float eps;
};

struct LinearBwdParams {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b, *W_ckpt, *W_last;
  const void* saved;  // per mini-batch values written by the forward (LinSavedSlot)
  void *dXQ, *dXK, *dXV, *deta;
  float *dW, *db, *dln_w, *dln_b;
  int B, H, NC, F, G, NK;
  int eta_rule;  // as the forward's; deta is then dlr [NC][K] fp32 unless dense
};

// What the TTT-Linear forward saves per mini-batch for the backward, one slot
// per (chain, mini-batch) in the saved buffer [B*H][NC][slot].  Byte offsets,
// fp32; tiles in lane order (each lane's 4 registers contiguous):
//   G    [F/16][64] x 4   inner-loss gradient, token-major C-layout tiles
//   XH   [F/16][64] x 4   normalised Z1 = XK W + b, token-major
//   XHB  [F/16][64] x 4   normalised readout Zb, feature-major (lane (g, n)
//                         holds features 16o + 4g + j of token n)
//   RSTD [16], CC [16]    per token: 1/sigma(Z1) and mean(gx * xh) of the
//                         inner-loss LayerNorm
//   RSB  [16]             per token: 1/sigma(Zb)
template <int F> struct LinSavedSlot {
  static constexpr int G = 0;
  static constexpr int XH = F * 64;
  static constexpr int XHB = 2 * F * 64;
  static constexpr int RSTD = 3 * F * 64;
  static constexpr int CC = RSTD + 64;
  static constexpr int RSB = CC + 64;
  static constexpr int BYTES = RSTD + 256;
};
constexpr size_t lin_saved_slot_bytes(int F) { return (size_t)3 * F * 64 + 256; }
size_t linear_saved_slot_bytes(int F);

struct MlpFwdParams {
  const void *XQ, *XK, *XV, *eta;
  const float *ln_w, *ln_b, *W1_init, *b1_init, *W2_init, *b2_init;
  void* out;
  float *W1_last, *b1_last, *W2_last, *b2_last;
  float *W1_ckpt, *b1_ckpt, *W2_ckpt, *b2_ckpt;
  float *W1_memo, *b1_memo, *W2_memo, *b2_memo;
  void* saved;  // per mini-batch values for the backward, MlpSavedSlot layout (may be null)
  int B, H, NC, F, FF, G, NK, M, NS;
  int eta_rule;  // TTT_ETA_*: eta dense [NC][K][K] (activation type) or lr [NC][K] fp32
  float eps;
};

struct MlpBwdParams {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b, *W1_ckpt, *b1_ckpt, *W2_ckpt, *b2_ckpt;
  const float *W1_last, *b1_last, *W2_last, *b2_last;
  const void* saved;  // per mini-batch values written by the forward
  void* ws;           // per mini-batch handoff from the reverse sweep to the dXQ/dXK pass (MlpBwdWsSlot)
  int* dx_ctrl;       // fused dXQ/dXK workers: [task counter, timeout flag, pad, pad, group flags [B*H][NK]];
                      // nullptr = a second launch after the sweep
  void *dXQ, *dXK, *dXV, *deta;
  float *dW1, *db1, *dW2, *db2, *dln_w, *dln_b;
  int B, H, NC, F, FF, G, NK;
  int eta_rule;      // as the forward's; deta is then dlr [NC][K] fp32 unless dense
  int dx_max_polls;  // fused dXQ/dXK workers: polls of a group flag before giving up
  int dx_fused;      // 0: the dXQ/dXK pass is always a second launch
  float eps;
};

struct MlpReadoutParams {
  const void* XQ;
  const float *W1, *b1, *W2, *b2, *ln_w, *ln_b;
  float* out;
  int B, H, ntok, F, FF, S, nchunk;
  float eps;
};

hipError_t launch_mlp_readout(const MlpReadoutParams& p, int dtype, hipStream_t stream);
int mlp_readout_chunk_tokens();

// Memory-cache combiner (ttt_layer.py:506-561): memo states [B,H,NS,...],
// gates buffer of memo_gate_floats_per_chain() floats per chain.
constexpr int kMemoMaxStates = 256;
struct MlpMemoParams {
  const void *XQ, *XK, *XU, *XQW, *dout;
  const float *W1, *b1, *W2, *b2, *ln_w, *ln_b;
  void *out, *dXK, *dXU, *dXQW;
  float* gates;
  unsigned char* packed;  // bf16: [B*H][NS] LDS images of the memo states (mlp_memo_image_bytes each), or null
  int B, H, NC, F, FF, M, NS, nchunk;
  float eps;
};
size_t memo_gate_floats_per_chain(int NC, int K, int F, int M);
size_t mlp_memo_image_bytes(int F, int FF);
hipError_t launch_mlp_memo(const MlpMemoParams& p, int dtype, bool bwd, hipStream_t stream);
int mlp_memo_chunk_tiles(int B, int H, int NC);  // mini-batches per combiner workgroup chunk

// What the TTT-MLP forward saves per mini-batch for the backward, one slot
// per (chain, mini-batch) in the saved buffer [B*H][NC][slot].  Byte offsets;
// ST = bytes of the activation type; "lane order" = each lane's registers
// stored contiguously, so a wave reads a tile back with one access per lane.
//   state update:
//     G1E [FF/64][4][64] x 4 ST   -e*G1 as W1-update operand frags, per 64-unit slice
//     G2E [F/16][64] x 4 ST       -e*G2 as W2-update operand frags
//     B1D [FF], B2D [F] fp32      bias decrements (b -= G^T e)
//   forward activations (token-major C-layout tiles, lane order), with
//   Z1 = XK W1 + b1, Pm = G2 W2^T and the readout's Z1b:
//     X2, SP1, G1, H1    [FF/64][4][64] x 4 ST   gelu(Z1) (the W2-update operand
//                        frags), gelu'(Z1), G1 = Pm gelu'(Z1), Pm gelu''(Z1)
//     X2B, SP1B          [FF/64][4][64] x 4 ST   gelu(Z1b), gelu'(Z1b)
//     G2, XH, XHB  [F/16][64] x 4 fp32     G2, normalised Z2, normalised Z2b
//     RSTD, CC, RSB [64] x 4 fp32          per-row 1/sigma(Z2), mean(gx * xh), 1/sigma(Z2b)
//     A2T [16][16] fp32 row-major          (X2b X2^T)^T
template <int F, int FF, int ST> struct MlpSavedSlot {
  static constexpr int G1E = 0;
  static constexpr int G2E = G1E + FF * 16 * ST;
  static constexpr int B1D = G2E + F * 16 * ST;
  static constexpr int B2D = B1D + FF * 4;
  static constexpr int X2 = B2D + F * 4;
  static constexpr int SP1 = X2 + FF * 16 * ST;
  static constexpr int G1 = SP1 + FF * 16 * ST;
  static constexpr int H1 = G1 + FF * 16 * ST;
  static constexpr int X2B = H1 + FF * 16 * ST;
  static constexpr int SP1B = X2B + FF * 16 * ST;
  static constexpr int G2 = SP1B + FF * 16 * ST;
  static constexpr int XH = G2 + F * 64;
  static constexpr int XHB = XH + F * 64;
  static constexpr int RSTD = XHB + F * 64;
  static constexpr int CC = RSTD + 1024;
  static constexpr int RSB = CC + 1024;
  static constexpr int A2T = RSB + 1024;
  static constexpr int BYTES = A2T + 1024;
};
constexpr size_t mlp_saved_slot_bytes_of(int F, int FF, int ST) {
  return (size_t)(7 * FF + F) * 16 * ST + (size_t)(FF + F) * 4 + (size_t)3 * F * 64 + 4 * 1024;
}

// The MLP backward's handoff per (chain, mini-batch) from its reverse sweep to
// the pass that forms dXQ and dXK (byte offsets, lane order):
//   DZ1BF, DZ1F [FF/64][4][64] x 4 ST   dZ1b and dZ1 as frags of [16 x FF] (free = token)
//   XQP, XKP    [F/16][64] x 4 fp32      the dXQ / dXK terms that do not involve W1
template <int F, int FF, int ST> struct MlpBwdWsSlot {
  static constexpr int DZ1BF = 0;
  static constexpr int DZ1F = FF * 16 * ST;
  static constexpr int XQP = 2 * FF * 16 * ST;
  static constexpr int XKP = XQP + F * 64;
  static constexpr int BYTES = XKP + F * 64;
};
size_t mlp_bwd_ws_slot_bytes(int F, int FF, int dtype);
// bytes of the control words after the B*H*NC handoff slots of the MLP backward workspace
size_t mlp_bwd_ctrl_bytes(int B, int H, int NC, int G);

hipError_t launch_mlp_bwd(const MlpBwdParams& p, int dtype, hipStream_t stream);
// bytes of one (chain, mini-batch) slot of the forward's saved buffer
size_t mlp_saved_slot_bytes(int F, int FF, int dtype);

hipError_t launch_mlp_fwd(const MlpFwdParams& p, int dtype, hipStream_t stream);

// Producer / consumer around the inner loop (ttt_layer_io.hip)
struct ProducerParams {
  const void* proj;  // [B*L][ld]: XQ | XK | XV | XU (H*F each) | H lr logits | padding
  int ld;
  const float *rope, *ln_w, *ln_b;  // rope [L][F/2][2] (cos, sin); ln [H][F]
  void *XQ, *XK, *XV, *XU;          // [B,H,L,F] (= [B,H,NC,K,F])
  float* lr;                        // [B,H,L]
  const void *dXQ, *dXK, *dXV, *dXU;
  const float* dlr;  // may be null
  void* dproj;       // [B*L][ld]
  float* partial;    // [blocks][2][H*F]: LN-parameter gradient partials
  int B, L, H, F;
  float base_lr, eps, l2eps;
};
struct PostNormParams {
  const void* X;  // [B,H,L,F]
  const float *gamma, *beta;
  void* Y;        // [B,L,H*F]
  float* stats;   // [B*L][2]: mean, 1/sigma
  const void* dY;
  void* dX;
  float* partial;  // [blocks][2][H*F]
  int B, L, H, F;
  float eps;
};
hipError_t launch_producer(const ProducerParams& p, int dtype, bool bwd, hipStream_t stream);
hipError_t launch_post_norm(const PostNormParams& p, int dtype, bool bwd, hipStream_t stream);
int layer_io_bwd_blocks(int B, int L);
int layer_io_max_width();

hipError_t launch_linear_fwd(const LinearFwdParams& p, int dtype, hipStream_t stream);
hipError_t launch_linear_fwd_rows(const LinearFwdParams& p, int dtype, hipStream_t stream);  // 16-bit activations
hipError_t launch_linear_bwd(const LinearBwdParams& p, int dtype, hipStream_t stream);

// ---- general-shape inner loops (ttt_generic.hip): K, F, FF multiples of 16
// outside the specialised kernels' set.  The `saved` buffer holds, per chain,
// the state entering every mini-batch and the per-mini-batch fp32 scratch
// (offsets in floats from the chain's block).
struct GenLayout {
  int K, F, FF, NC;
  bool mlp;
  size_t state;  // floats of one state (W1, b1[, W2, b2]), padded to 4
  size_t states, wfin;
  size_t xq, xk, xv, dout, eta, a1, c1, a2, c2, deta, da1, dc1, da2, dc2;
  size_t z1, x2, d1, dd1, p, g1, z1b, x2b, db;
  size_t z2, z2h, g2, z2b, z2bh, sig2, sigb, de;
  size_t t1, dg1, dx2, dx2b, dz1b, dp, dz1, t2, dg2, dz2b, dz2, dxq, dxk, dxv, lnwt, lnbt;
  size_t per_chain;
  __host__ __device__ GenLayout(int K, int F, int FF, int NC, bool mlp);
};
struct GenFwdParams {
  const void *XQ, *XK, *XV, *eta;
  const float *ln_w, *ln_b, *W1_init, *b1_init, *W2_init, *b2_init;
  void* out;
  float *W1_last, *b1_last, *W2_last, *b2_last;
  float *W1_ckpt, *b1_ckpt, *W2_ckpt, *b2_ckpt;
  float *W1_memo, *b1_memo, *W2_memo, *b2_memo;
  void* saved;
  int B, H, NC, K, F, FF, G, M, eta_rule;
  bool mlp;
  float eps;
};
struct GenBwdParams {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b;
  void *dXQ, *dXK, *dXV, *deta;
  float *dW1, *db1, *dW2, *db2, *dln_w, *dln_b;
  void* saved;  // written by the forward with the same shapes
  void* ws;     // the backward's workspace (the register-resident MLP backward's handoff), may be null
  size_t ws_bytes;
  int B, H, NC, K, F, FF, eta_rule;
  bool mlp;
  float eps;
};
bool gen_shape_ok(int K, int F, int FF, bool mlp);
size_t gen_saved_bytes(int B, int H, int NC, int K, int F, int FF, bool mlp);
hipError_t launch_gen_fwd(const GenFwdParams& p, int dtype, hipStream_t stream);
hipError_t launch_gen_bwd(const GenBwdParams& p, int dtype, hipStream_t stream);
// register-resident kernels (ttt_small.hip) for the general-shape set's small
// heads: K = 16..64, F = 32 (and FF = 32), one wavefront per chain, same
// interface and saved-buffer layout (only the states of GenLayout are used)
bool small_shape_ok(int K, int F, int FF, bool mlp);
// workspace bytes of the register-resident MLP backward's two-launch form
// (0 for K outside 16..64); a smaller workspace runs the one-launch form
size_t small_mlp_bwd_hand_bytes(int B, int H, int NC, int K);
bool gen_force_general();  // TTT_OPT_SMALL_KERNELS = 0: always the staged general-shape kernels
hipError_t launch_small_fwd(const GenFwdParams& p, int dtype, hipStream_t stream);
hipError_t launch_small_bwd(const GenBwdParams& p, int dtype, hipStream_t stream);

}  // namespace ttt
