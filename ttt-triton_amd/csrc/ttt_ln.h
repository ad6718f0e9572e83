// LayerNorm pieces on register tiles.
//
// Token-major ("TM") rows: a [16 x 16*FT] matrix held as FT C-layout tiles;
// row t = 4g + j lives in register j of the 16 lanes of group g, across the
// FT tiles, so a row reduction is an in-lane sum over tiles plus a DPP sum
// over 16 lanes.
//
// Feature-major ("FM") rows: the transpose, [16*FT x 16] as FT tiles; token
// t = n lives in lanes n, n+16, n+32, n+48 with features in registers, so a
// token reduction is an in-lane sum over 4*FT values plus two lane swaps.
#pragma once

#include "ttt_tile.h"

namespace ttt {

// ln_fused_l2_bwd (ops/ttt_utils.py:21-48) on TM rows, keeping what its
// backward needs.  z: pre-LN values, tgt: reconstruction target.
template <int FT> struct LnL2TM {
  f4 rstd;        // 1/sqrt(var + eps) per row j
  f4 c;           // mean(gx * xh) per row j
  f4 xh[FT];      // normalised z
  f4 go[FT];      // gamma*xh + beta - tgt
  f4 gx[FT];      // go * gamma

  __device__ __forceinline__ void forward(const Tile (&z)[FT], const f4 (&tgt)[FT], const float (&lnw)[FT],
                                          const float (&lnb)[FT], float eps, Tile (&G)[FT]) {
    constexpr float invF = 1.0f / (16 * FT);
    f4 mu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o) s += z[o].v[j];
      mu[j] = sum_row16(s) * invF;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const float d = z[o].v[j] - mu[j];
        s += d * d;
      }
      rstd[j] = rsqrt_f(sum_row16(s) * invF + eps);
    }
    f4 s1 = f4{0.f, 0.f, 0.f, 0.f}, s2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xh[o][j] = (z[o].v[j] - mu[j]) * rstd[j];
        go[o][j] = lnw[o] * xh[o][j] + lnb[o] - tgt[o][j];
        gx[o][j] = go[o][j] * lnw[o];
        s1[j] += gx[o][j];
        s2[j] += gx[o][j] * xh[o][j];
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s1[j] = sum_row16(s1[j]) * invF;
      c[j] = sum_row16(s2[j]) * invF;
    }
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) G[o].v[j] = (gx[o][j] - s1[j] - xh[o][j] * c[j]) * rstd[j];
  }

  // Backward of G = ln_fused_l2_bwd(z, tgt): given dG, returns dz and dtgt
  // and accumulates the per-lane LN-parameter gradient partials (row sums
  // over the 4 rows this lane holds; the caller sums over lane groups).
  __device__ __forceinline__ void backward(const Tile (&dG)[FT], const Tile (&G)[FT], const float (&lnw)[FT],
                                           f4 (&dz)[FT], f4 (&dtgt)[FT], float (&dlnw)[FT], float (&dlnb)[FT]) const {
    constexpr float invF = 1.0f / (16 * FT);
    f4 u[FT];
    f4 mu_u = f4{0.f, 0.f, 0.f, 0.f}, mu_ux = f4{0.f, 0.f, 0.f, 0.f}, dsig = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u[o][j] = dG[o].v[j] * rstd[j];
        mu_u[j] += u[o][j];
        mu_ux[j] += u[o][j] * xh[o][j];
        dsig[j] += u[o][j] * G[o].v[j];
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mu_u[j] = sum_row16(mu_u[j]) * invF;
      mu_ux[j] = sum_row16(mu_ux[j]) * invF;
      dsig[j] = -sum_row16(dsig[j]);
    }
    f4 dxh[FT];
    f4 m1 = f4{0.f, 0.f, 0.f, 0.f}, m2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      float aw = 0.f, ab = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float d_gx = u[o][j] - mu_u[j] - xh[o][j] * mu_ux[j];
        const float d_go = d_gx * lnw[o];
        aw += d_gx * go[o][j] + d_go * xh[o][j];
        ab += d_go;
        dtgt[o][j] = -d_go;
        dxh[o][j] = -c[j] * u[o][j] - mu_ux[j] * gx[o][j] + d_go * lnw[o];
        m1[j] += dxh[o][j];
        m2[j] += dxh[o][j] * xh[o][j];
      }
      dlnw[o] += aw;
      dlnb[o] += ab;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m1[j] = sum_row16(m1[j]) * invF;
      m2[j] = sum_row16(m2[j]) * invF;
    }
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dz[o][j] = rstd[j] * (dxh[o][j] - m1[j] - xh[o][j] * m2[j]) + dsig[j] * xh[o][j] * invF;
  }
};

// The same function as LnL2TM keeping only rstd, c and xh between forward and
// backward (16 + 8 registers per lane at F = 64 instead of 56); the backward
// recomputes gamma*xh + beta - tgt from xh and the target.
template <int FT> struct LnL2Lite {
  f4 rstd;    // 1/sqrt(var + eps) per row j
  f4 c;       // mean(gx * xh) per row j
  f4 xh[FT];  // normalised z

  __device__ __forceinline__ void forward(const Tile (&z)[FT], const f4 (&tgt)[FT], const float (&lnw)[FT],
                                          const float (&lnb)[FT], float eps, Tile (&G)[FT]) {
    constexpr float invF = 1.0f / (16 * FT);
    f4 mu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o) s += z[o].v[j];
      mu[j] = sum_row16(s) * invF;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const float d = z[o].v[j] - mu[j];
        s += d * d;
      }
      rstd[j] = rsqrt_f(sum_row16(s) * invF + eps);
    }
    f4 gx[FT];
    f4 s1 = f4{0.f, 0.f, 0.f, 0.f}, s2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xh[o][j] = (z[o].v[j] - mu[j]) * rstd[j];
        gx[o][j] = (lnw[o] * xh[o][j] + lnb[o] - tgt[o][j]) * lnw[o];
        s1[j] += gx[o][j];
        s2[j] += gx[o][j] * xh[o][j];
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s1[j] = sum_row16(s1[j]) * invF;
      c[j] = sum_row16(s2[j]) * invF;
    }
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) G[o].v[j] = (gx[o][j] - s1[j] - xh[o][j] * c[j]) * rstd[j];
  }

  __device__ __forceinline__ void backward(const Tile (&dG)[FT], const Tile (&G)[FT], const f4 (&tgt)[FT],
                                           const float (&lnw)[FT], const float (&lnb)[FT], f4 (&dz)[FT],
                                           f4 (&dtgt)[FT], float (&dlnw)[FT], float (&dlnb)[FT]) const {
    constexpr float invF = 1.0f / (16 * FT);
    f4 u[FT];
    f4 mu_u = f4{0.f, 0.f, 0.f, 0.f}, mu_ux = f4{0.f, 0.f, 0.f, 0.f}, dsig = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u[o][j] = dG[o].v[j] * rstd[j];
        mu_u[j] += u[o][j];
        mu_ux[j] += u[o][j] * xh[o][j];
        dsig[j] += u[o][j] * G[o].v[j];
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mu_u[j] = sum_row16(mu_u[j]) * invF;
      mu_ux[j] = sum_row16(mu_ux[j]) * invF;
      dsig[j] = -sum_row16(dsig[j]);
    }
    f4 dxh[FT];
    f4 m1 = f4{0.f, 0.f, 0.f, 0.f}, m2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      float aw = 0.f, ab = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float go = lnw[o] * xh[o][j] + lnb[o] - tgt[o][j];
        const float gx = go * lnw[o];
        const float d_gx = u[o][j] - mu_u[j] - xh[o][j] * mu_ux[j];
        const float d_go = d_gx * lnw[o];
        aw += d_gx * go + d_go * xh[o][j];
        ab += d_go;
        dtgt[o][j] = -d_go;
        dxh[o][j] = -c[j] * u[o][j] - mu_ux[j] * gx + d_go * lnw[o];
        m1[j] += dxh[o][j];
        m2[j] += dxh[o][j] * xh[o][j];
      }
      dlnw[o] += aw;
      dlnb[o] += ab;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m1[j] = sum_row16(m1[j]) * invF;
      m2[j] = sum_row16(m2[j]) * invF;
    }
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dz[o][j] = rstd[j] * (dxh[o][j] - m1[j] - xh[o][j] * m2[j]) + dsig[j] * xh[o][j] * invF;
  }
};

// LayerNorm statistics of FM tiles (one token per lane column).
template <int FT> __device__ __forceinline__ void ln_stats_fm(const Tile (&z)[FT][1], float eps, float& mean,
                                                              float& rstd) {
  constexpr float invF = 1.0f / (16 * FT);
  float s = 0.f;
#pragma unroll
  for (int o = 0; o < FT; ++o)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += z[o][0].v[j];
  mean = sum_col4(s) * invF;
  float v = 0.f;
#pragma unroll
  for (int o = 0; o < FT; ++o)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = z[o][0].v[j] - mean;
      v += d * d;
    }
  rstd = rsqrt_f(sum_col4(v) * invF + eps);
}

}  // namespace ttt
