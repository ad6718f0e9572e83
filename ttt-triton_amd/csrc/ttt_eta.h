// The per-mini-batch eta of the dual form, from either of its two sources.
//
// Dense: eta [NC][K][K] in the activation type, as ops/ttt_linear.py and
// ops/ttt_mlp.py take it, and its gradient deta of the same shape.
//
// Learning-rate vector: lr [NC][K] fp32 (what TTTBase.get_eta returns per
// token, ttt_layer.py:151-163) and a rule that expands it on chip:
//   TTT_ETA_LAYER   eta[i][j] = lr[j] / K for every row i  (ttt_layer.py:309)
//   TTT_ETA_CAUSAL  eta[i][j] = lr[j] / (i + 1) for j <= i, else 0
// The gradient is then dlr[j] = sum_i deta[i][j] * coef(i, j), fp32.  The
// coefficients are formed as the host forms them (1/K, or 1/(i+1) rounded to
// fp32, times lr), so a dense fp32 eta built from the same lr gives
// bit-identical eta values.
#pragma once

#include "../../include/ttt_amd.h"
#include "ttt_buf.h"

namespace ttt {

constexpr int kEtaK = 16;

// coefficient of lr[j] in eta[i][j] under `rule` (wave-uniform)
__device__ __forceinline__ float eta_coef(int rule, int i, int j) {
  if (rule == TTT_ETA_LAYER) return 1.0f / kEtaK;
  return j <= i ? 1.0f / (float)(i + 1) : 0.0f;
}

// lane (g, n) of a frag laid out as eta[n][4g + j] (row n, columns 4g..4g+3):
// the 4 values from lr4 = lr[4g .. 4g+3]
__device__ __forceinline__ f4 eta_rowfrag_from_lr(int rule, f4 lr4) {
  const int l = lane_id(), g = l >> 4, n = l & 15;
  f4 e;
  if (rule == TTT_ETA_LAYER) {
    e = lr4 * (1.0f / kEtaK);
  } else {
    const float c = 1.0f / (float)(n + 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) e[j] = 4 * g + j <= n ? lr4[j] * c : 0.0f;
  }
  return e;
}

// lane (g, n) of a C-layout tile eta[4g + j][n]: from lr[n]
__device__ __forceinline__ f4 eta_ctile_from_lr(int rule, float lrn) {
  const int l = lane_id(), g = l >> 4, n = l & 15;
  f4 e;
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = lrn * eta_coef(rule, 4 * g + j, n);
  return e;
}

// last row: eta[K-1][4g + j] = lr[4g + j] / K under both rules
__device__ __forceinline__ f4 eta_lastrow_from_lr(f4 lr4) { return lr4 * (1.0f / kEtaK); }

// dlr contribution of a deta frag held as deta[n][4g + j] (lane (g, n)):
// sum over the rows n of deta * coef, the same in all 16 lanes of group g
__device__ __forceinline__ f4 dlr_from_detaT(int rule, f4 detT) {
  const int l = lane_id(), g = l >> 4, n = l & 15;
  f4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = sum_row16(detT[j] * eta_coef(rule, n, 4 * g + j));
  return r;
}

}  // namespace ttt
