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
  int B, H, NC, F, FF, G, NK, M, NS;
  float eps;
};

struct MlpBwdParams {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b, *W1_ckpt, *b1_ckpt, *W2_ckpt, *b2_ckpt;
  void *dXQ, *dXK, *dXV, *deta;
  float *dW1, *db1, *dW2, *db2, *dln_w, *dln_b;
  void* ws;  // per-chain: G slots of the state's operand values
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

hipError_t launch_mlp_bwd(const MlpBwdParams& p, int dtype, hipStream_t stream);
size_t mlp_bwd_slot_bytes(int F, int FF, int dtype);

hipError_t launch_mlp_fwd(const MlpFwdParams& p, int dtype, hipStream_t stream);

hipError_t launch_linear_fwd(const LinearFwdParams& p, int dtype, hipStream_t stream);
hipError_t launch_linear_bwd(const LinearBwdParams& p, int dtype, hipStream_t stream);

}  // namespace ttt
