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
  int B, H, NC, F, G, NK;
  float eps;
};

struct LinearBwdParams {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b, *W_ckpt, *b_ckpt;
  void *dXQ, *dXK, *dXV, *deta;
  float *dW, *db, *dln_w, *dln_b;
  float* ws;  // per-chain scratch: G mini-batches of the inner-loss gradient
  int B, H, NC, F, G, NK;
  float eps;
};

struct MlpFwdParams {
  const void *XQ, *XK, *XV, *eta;
  const float *ln_w, *ln_b, *W1_init, *b1_init, *W2_init, *b2_init;
  void* out;
  float *W1_last, *b1_last, *W2_last, *b2_last;
  float *W1_ckpt, *b1_ckpt, *W2_ckpt, *b2_ckpt;
  float *W1_memo, *b1_memo, *W2_memo, *b2_memo;
  void* upd;  // per mini-batch update operands for the backward (may be null)
  int B, H, NC, F, FF, G, NK, M, NS;
  float eps;
};

struct MlpBwdParams {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b, *W1_ckpt, *b1_ckpt, *W2_ckpt, *b2_ckpt;
  const float *W1_last, *b1_last, *W2_last, *b2_last;
  const void* upd;  // update operands written by the forward
  void *dXQ, *dXK, *dXV, *deta;
  float *dW1, *db1, *dW2, *db2, *dln_w, *dln_b;
  int B, H, NC, F, FF, G, NK;
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

// One mini-batch's TTT-MLP update operands in the upd buffer [B*H][NC][slot]
// (byte offsets; ST = bytes of the activation type):
//   g1e [FF/64][4][64] x 4 ST   -e*G1, the W1-update MFMA operand frags per 64-unit slice
//   g2e [F/16][64] x 4 ST       -e*G2, the W2-update MFMA operand frags
//   b1d [FF] fp32, b2d [F] fp32  bias decrements (b -= G^T e)
template <int F, int FF, int ST> struct MlpUpdSlot {
  static constexpr int G1E = 0;
  static constexpr int G2E = FF * 16 * ST;
  static constexpr int B1D = (FF + F) * 16 * ST;
  static constexpr int B2D = B1D + FF * 4;
  static constexpr int BYTES = B2D + F * 4;
};

hipError_t launch_mlp_bwd(const MlpBwdParams& p, int dtype, hipStream_t stream);
// bytes of one mini-batch's update operands (per chain) in the forward's upd buffer
size_t mlp_upd_slot_bytes(int F, int FF, int dtype);

hipError_t launch_mlp_fwd(const MlpFwdParams& p, int dtype, hipStream_t stream);

hipError_t launch_linear_fwd(const LinearFwdParams& p, int dtype, hipStream_t stream);
hipError_t launch_linear_bwd(const LinearBwdParams& p, int dtype, hipStream_t stream);

}  // namespace ttt
