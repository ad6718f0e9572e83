// TTT-Linear backward on gfx950: one workgroup of two wavefronts per
// (batch, head) chain.
//
// Reverse sweep over checkpoint groups (kernels/linear_backward.py:278 walks
// the same groups; the algorithm here is our own):
//   phase 1  (wave 0) reload W, b from the checkpoint entering the group, run
//            the group's mini-batches forward computing only the inner-loss
//            gradient G_s = ln_fused_l2_bwd(XK_s W_s + b_s, XV_s - XK_s), park
//            G_s in the per-chain workspace, and apply the state update;
//   phase 2  walk the group backwards.  Wave 0 owns the fast weight: it
//            rebuilds the state entering mini-batch s from the one after it,
//            W_s = W_{s+1} + XK_s^T diag(e_s) G_s (the forward's MFMA operands),
//            recomputes the mini-batch forward and applies its gradient
//            (ops/ttt_linear.py:8-54 differentiated by hand).  Wave 1 owns the
//            gradient wrt the state, dW and db: per mini-batch it first
//            produces XK dW' + db' and -(e G) dW'^T, which wave 0 needs, and
//            after wave 0 has the mini-batch's dZb and dZ1 it applies
//            dW += XQ^T dZb + XK^T dZ1.  Two barriers per mini-batch; wave 0's
//            recompute of mini-batch s-1 overlaps wave 1's work on s.
// Products that contract W or dW over their column index use operand frags
// transposed exactly with identity MFMAs, so neither wave keeps a transposed
// copy of its 16*F*F-byte state.
#include "ttt_kernels.h"
#include "ttt_ln.h"

namespace ttt {

template <typename T, int FT> struct LinBwdShared {
  float vlds[16 * FT];                 // wave 0: b in feature-major reads
  float lnacc[2][4 * FT][64];          // wave 0: readout-LN gradient partials per lane
  float dbz[16 * FT];                  // wave 0: column sums of dZb for the current step
  float red[2 * 16 * FT];              // wave 0: final reductions
  f4 qd[FT][64];                       // wave 1 -> 0: XK dW' + db'   (token-major tiles)
  f4 tr[FT][64];                       // wave 1 -> 0: -(e G) dW'^T   (token-major tiles)
  Frag<T> xq[2][FT][64];               // wave 0 -> 1: XQ token-major frags (by step parity)
  Frag<T> xk[2][FT][64];               // wave 0 -> 1: XK token-major frags
  Frag<T> dzb[2][FT][64];              // wave 0 -> 1: dZb token-major frags
  Frag<T> dz1[FT][64];                 // wave 0 -> 1: dZ1 token-major frags
  float db[16 * FT];                   // wave 0 -> 1: column sums of dZb + dZ1
  f4 dxq[FT][64];                      // wave 0: dXQ partial carried across the barrier
  float lnw[16 * FT];                  // wave 0: LN weight of this head
};

template <typename T, int FT> struct LinBwdCtx {
  const T *XQ, *XK, *XV, *DO, *ETA;
  T *DXQ, *DXK, *DXV, *DETA;
  float* WS;
  int NC, G, NK, chain, h;
};

// ------------------------------------------------------------------ wave 0
template <typename T, int FT> struct Wave0 {
  static constexpr int F = 16 * FT;
  static constexpr int K = 16;
  const LinearBwdParams& p;
  const LinBwdCtx<T, FT>& c;
  LinBwdShared<T, FT>& sh;
  int l, g, n;
  float eps;
  Frag<T> I;
  float lnw_tm[FT], lnb_tm[FT];
  float dlnw_tm[FT], dlnb_tm[FT];
  Tile W[FT][FT];
  float b_tm[FT];
  // carried from the first half of a step to the second
  Tile dG[FT], dxk[1][FT];
  f4 e, detT;
  Frag<T> dZbF[1][FT];
  LnL2TM<FT> ln;

  __device__ Wave0(const LinearBwdParams& p_, const LinBwdCtx<T, FT>& c_, LinBwdShared<T, FT>& sh_)
      : p(p_), c(c_), sh(sh_) {
    l = lane_id();
    g = l >> 4;
    n = l & 15;
    eps = p.eps;
    I = identity_frag<T>();
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      lnw_tm[o] = p.ln_w[c.h * F + 16 * o + n];
      lnb_tm[o] = p.ln_b[c.h * F + 16 * o + n];
      dlnw_tm[o] = 0.f;
      dlnb_tm[o] = 0.f;
    }
    for (int q = 0; q < 4 * FT; ++q) {
      sh.lnacc[0][q][l] = 0.f;
      sh.lnacc[1][q][l] = 0.f;
    }
    for (int f = l; f < F; f += 64) sh.lnw[f] = p.ln_w[c.h * F + f];
  }

  // phase 1: forward through mini-batches [s0, s1), parking G_s
  __device__ void recompute_group(int kk, int s0, int s1) {
    const float* wc = p.W_ckpt + ((size_t)c.chain * c.NK + kk) * F * F;
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) W[i][o] = load_tile(wc, F, 16 * i, 16 * o);
#pragma unroll
    for (int o = 0; o < FT; ++o) b_tm[o] = p.b_ckpt[((size_t)c.chain * c.NK + kk) * F + 16 * o + n];

    for (int s = s0; s < s1; ++s) {
      const T* xks = c.XK + (size_t)s * K * F;
      const T* xvs = c.XV + (size_t)s * K * F;
      Frag<T> xk[1][FT], xkTf[FT];
      f4 tgt[FT];
#pragma unroll
      for (int q = 0; q < FT; ++q) {
        xk[0][q] = load_frag(xks, F, 16 * q);
        const Tile xkT = transpose16(xk[0][q], I);
        xkTf[q] = to_frag<T>(xkT.v);
        tgt[q] = transpose16(load_frag(xvs, F, 16 * q), I).v - xkT.v;
      }
      const f4 ee = load4(c.ETA + (size_t)s * K * K + (K - 1) * K + 4 * g);
      Tile z1[1][FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) z1[0][o].v = f4{b_tm[o], b_tm[o], b_tm[o], b_tm[o]};
      gemm_pt<1, FT, FT>(z1, xk, W);
      LnL2TM<FT> l1;
      Tile Gs[FT];
      l1.forward(z1[0], tgt, lnw_tm, lnb_tm, eps, Gs);
      float* slot = c.WS + (size_t)(s - s0) * K * F;
#pragma unroll
      for (int o = 0; o < FT; ++o) spill_tile(slot + o * 256, Gs[o]);
      Frag<T> ge[FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        f4 v;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = -ee[j] * Gs[o].v[j];
          acc += ee[j] * Gs[o].v[j];
        }
        ge[o] = to_frag<T>(v);
        b_tm[o] -= sum_col4(acc);
      }
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) mma16(W[i][o].v, xkTf[i], ge[o]);
    }
  }

  // first half of the reverse step: rebuild the state entering s, recompute
  // the forward, readout-LN backward, everything that does not need dW'
  __device__ void step_a(int s, int s0) {
    const size_t xo = (size_t)s * K * F;
    const T* etas = c.ETA + (size_t)s * K * K;
    const int par = s & 1;
    Frag<T> xq[1][FT], xk[1][FT], dof[1][FT], xqTf[FT], xkTf[FT];
    f4 tgt[FT];
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      xq[0][q] = load_frag(c.XQ + xo, F, 16 * q);
      xk[0][q] = load_frag(c.XK + xo, F, 16 * q);
      dof[0][q] = load_frag(c.DO + xo, F, 16 * q);
      xqTf[q] = to_frag<T>(transpose16(xq[0][q], I).v);
      const Tile xkT = transpose16(xk[0][q], I);
      xkTf[q] = to_frag<T>(xkT.v);
      tgt[q] = transpose16(load_frag(c.XV + xo, F, 16 * q), I).v - xkT.v;
      sh.xq[par][q][l] = xqTf[q];
      sh.xk[par][q][l] = xkTf[q];
    }
    const f4 etaT = load_f4(etas, K, 0);  // [t_k x t_q]: eta[n][4g+j]
    f4 eta_n;                             // [t_q x t_k]: eta[4g+j][n]
#pragma unroll
    for (int j = 0; j < 4; ++j) eta_n[j] = (float)etas[(4 * g + j) * K + n];
    e = load4(etas + (K - 1) * K + 4 * g);

    Tile Gt[FT];
    {
      const float* slot = c.WS + (size_t)(s - s0) * K * F;
#pragma unroll
      for (int o = 0; o < FT; ++o) Gt[o] = fill_tile(slot + o * 256);
    }
    // rebuild the state entering s: W += XK^T (e G), b += G^T e
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      f4 v;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = e[j] * Gt[o].v[j];
        acc += v[j];
      }
      const Frag<T> eg = to_frag<T>(v);
#pragma unroll
      for (int i = 0; i < FT; ++i) mma16(W[i][o].v, xkTf[i], eg);
      b_tm[o] += sum_col4(acc);
      if (g == 0) sh.vlds[16 * o + n] = b_tm[o];
    }

    // recompute the mini-batch forward
    {
      Tile z1[1][FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) z1[0][o].v = f4{b_tm[o], b_tm[o], b_tm[o], b_tm[o]};
      gemm_pt<1, FT, FT>(z1, xk, W);
      Tile Gre[FT];
      ln.forward(z1[0], tgt, lnw_tm, lnb_tm, eps, Gre);
    }
    Tile at[1][1], a[1][1];
    at[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
    a[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
    gemm<1, 1, FT>(at, xk, xq);  // A^T [t_k x t_q]
    gemm<1, 1, FT>(a, xq, xk);   // A   [t_q x t_k]
    f4 mT, m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mT[j] = etaT[j] * at[0][0].v[j] + etaT[j];
      m[j] = eta_n[j] * a[0][0].v[j] + eta_n[j];
    }
    Tile zb[FT][1];
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) zb[o][0].v[j] = sh.vlds[16 * o + 4 * g + j];
    gemm_tp<FT, 1, FT>(zb, W, xq);
    {
      const Frag<T> mtf = to_frag<T>(mT);
#pragma unroll
      for (int o = 0; o < FT; ++o) mma16(zb[o][0].v, to_frag<T>(-Gt[o].v), mtf);
    }
    float mb, rsb;
    ln_stats_fm<FT>(zb, eps, mb, rsb);

    // readout LayerNorm backward (feature-major)
    Frag<T> dZbTf[FT];
    {
      constexpr float invF = 1.0f / F;
      f4 xhb[FT], gy[FT];
      float a1 = 0.f, a2 = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const f4 d = frag_to_f4(dof[0][o]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xhb[o][j] = (zb[o][0].v[j] - mb) * rsb;
          gy[o][j] = d[j] * sh.lnw[16 * o + 4 * g + j];
          sh.lnacc[0][4 * o + j][l] += d[j] * xhb[o][j];
          sh.lnacc[1][4 * o + j][l] += d[j];
          a1 += gy[o][j];
          a2 += gy[o][j] * xhb[o][j];
        }
      }
      a1 = sum_col4(a1) * invF;
      a2 = sum_col4(a2) * invF;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        f4 dz;
#pragma unroll
        for (int j = 0; j < 4; ++j) dz[j] = rsb * (gy[o][j] - a1 - xhb[o][j] * a2);
        dZbF[0][o] = to_frag<T>(dz);
        dZbTf[o] = to_frag<T>(transpose16(dZbF[0][o], I).v);
        sh.dzb[par][o][l] = dZbTf[o];
        // column sums over tokens (fp32) for db
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float cs = sum_row16(dz[j]);
          if (n == 0) sh.dbz[16 * o + 4 * g + j] = cs;
        }
      }
    }

    // dXQ = dout + dA XK (+ dZb W^T later); dM = -dZb G^T; dA = dM (.) eta
    Tile dxq[1][FT];
#pragma unroll
    for (int q = 0; q < FT; ++q) dxq[0][q] = transpose16(dof[0][q], I);
    {
      Frag<T> GF[1][FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) GF[0][o] = to_frag<T>(transpose16(to_frag<T>(Gt[o].v), I).v);
      Tile dm[1][1], dmT[1][1];
      dm[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      dmT[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      gemm<1, 1, FT>(dm, dZbF, GF);   // dZb G^T  [t_q x t_k]
      gemm<1, 1, FT>(dmT, GF, dZbF);  // G dZb^T  [t_k x t_q]
      f4 daT, da;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        detT[j] = -dmT[0][0].v[j] * (1.0f + at[0][0].v[j]);
        daT[j] = -dmT[0][0].v[j] * etaT[j];
        da[j] = -dm[0][0].v[j] * eta_n[j];
      }
      const Frag<T> daTf = to_frag<T>(daT), daf = to_frag<T>(da);
      const Frag<T> mf = to_frag<T>(-m);
#pragma unroll
      for (int q = 0; q < FT; ++q) {
        mma16(dxq[0][q].v, daTf, xkTf[q]);  // dA XK
        dxk[0][q].v = f4{0.f, 0.f, 0.f, 0.f};
        mma16(dxk[0][q].v, daf, xqTf[q]);   // dA^T XQ
        dG[q].v = f4{0.f, 0.f, 0.f, 0.f};
        mma16(dG[q].v, mf, dZbTf[q]);       // -M^T dZb
        sh.dxq[q][l] = dxq[0][q].v;
      }
    }
  }

  // second half: needs XK dW' + db' and -(e G) dW'^T from wave 1
  __device__ void step_b(int s, int s0) {
    const size_t xo = (size_t)s * K * F;
    Tile Gt[FT], dxq[1][FT];
    {
      const float* slot = c.WS + (size_t)(s - s0) * K * F;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        Gt[o] = fill_tile(slot + o * 256);
        dxq[0][o].v = sh.dxq[o][l];
      }
    }
    float de[4] = {0.f, 0.f, 0.f, 0.f};
    {
      f4 dep = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const f4 qd = sh.qd[o][l];
        dxk[0][o].v += sh.tr[o][l];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dG[o].v[j] -= e[j] * qd[j];
          dep[j] += Gt[o].v[j] * qd[j];
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) de[j] = -sum_row16(dep[j]);
    }
    f4 dz1[FT], dtgt[FT];
    ln.backward(dG, Gt, lnw_tm, dz1, dtgt, dlnw_tm, dlnb_tm);
    Frag<T> dz1F[1][FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      const Frag<T> f = to_frag<T>(dz1[o]);
      sh.dz1[o][l] = f;
      dz1F[0][o] = to_frag<T>(transpose16(f, I).v);
      dxk[0][o].v -= dtgt[o];
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc += dz1[o][j];
      acc = sum_col4(acc);
      if (g == 0) sh.db[16 * o + n] = acc + sh.dbz[16 * o + n];
    }
    // dZb W^T into dXQ and dZ1 W^T into dXK, one transposed W block at a time
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int q = 0; q < FT; q += 2) {
        const Frag<T> t0 = to_frag<T>(transpose16(to_frag<T>(W[i][q].v), I).v);
        const Frag<T> t1 = to_frag<T>(transpose16(to_frag<T>(W[i][q + 1].v), I).v);
        mma32(dxq[0][i].v, dZbF[0][q], dZbF[0][q + 1], t0, t1);
        mma32(dxk[0][i].v, dz1F[0][q], dz1F[0][q + 1], t0, t1);
      }
    // write the mini-batch's gradients (feature-major: 4 contiguous elements per lane)
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      store_f4(c.DXQ + xo, F, 16 * q, transpose16(to_frag<T>(dxq[0][q].v), I).v);
      store_f4(c.DXK + xo, F, 16 * q, transpose16(to_frag<T>(dxk[0][q].v), I).v);
      store_f4(c.DXV + xo, F, 16 * q, transpose16(to_frag<T>(dtgt[q]), I).v);
    }
    if (n == K - 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) detT[j] += de[j];
    }
    store_f4(c.DETA + (size_t)s * K * K, K, 0, detT);
  }

  __device__ void finish() {
    float lw_t[FT], lb_t[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      lw_t[o] = sum_col4(dlnw_tm[o]);
      lb_t[o] = sum_col4(dlnb_tm[o]);
    }
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float w = sum_row16(sh.lnacc[0][4 * o + j][l]);
        const float b = sum_row16(sh.lnacc[1][4 * o + j][l]);
        if (n == 0) {
          sh.red[16 * o + 4 * g + j] = w;
          sh.red[F + 16 * o + 4 * g + j] = b;
        }
      }
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        p.dln_w[(size_t)c.chain * F + 16 * o + n] = lw_t[o] + sh.red[16 * o + n];
        p.dln_b[(size_t)c.chain * F + 16 * o + n] = lb_t[o] + sh.red[F + 16 * o + n];
      }
    }
  }
};

// ------------------------------------------------------------------ wave 1
template <typename T, int FT> struct Wave1 {
  static constexpr int F = 16 * FT;
  static constexpr int K = 16;
  const LinearBwdParams& p;
  const LinBwdCtx<T, FT>& c;
  LinBwdShared<T, FT>& sh;
  int l, g, n;
  Frag<T> I;
  Tile dW[FT][FT];
  float db_tm[FT];

  __device__ Wave1(const LinearBwdParams& p_, const LinBwdCtx<T, FT>& c_, LinBwdShared<T, FT>& sh_)
      : p(p_), c(c_), sh(sh_) {
    l = lane_id();
    g = l >> 4;
    n = l & 15;
    I = identity_frag<T>();
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) dW[i][o].v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o) db_tm[o] = 0.f;
  }

  // XK dW' + db' and -(e G) dW'^T for mini-batch s (dW' = gradient after s)
  __device__ void carry_terms(int s, int s0) {
    const T* xks = c.XK + (size_t)s * K * F;
    Frag<T> xk[1][FT];
#pragma unroll
    for (int q = 0; q < FT; ++q) xk[0][q] = load_frag(xks, F, 16 * q);
    const f4 e = load4(c.ETA + (size_t)s * K * K + (K - 1) * K + 4 * g);
    const float* slot = c.WS + (size_t)(s - s0) * K * F;
    Frag<T> eGF[1][FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      const Tile gt = fill_tile(slot + o * 256);
      f4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = e[j] * gt.v[j];
      eGF[0][o] = to_frag<T>(-transpose16(to_frag<T>(v), I).v);
    }
    Tile qm[1][FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) qm[0][o].v = f4{db_tm[o], db_tm[o], db_tm[o], db_tm[o]};
    gemm_pt<1, FT, FT>(qm, xk, dW);
#pragma unroll
    for (int o = 0; o < FT; ++o) sh.qd[o][l] = qm[0][o].v;
#pragma unroll
    for (int i = 0; i < FT; ++i) {
      Tile t;
      t.v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < FT; q += 2) {
        const Frag<T> t0 = to_frag<T>(transpose16(to_frag<T>(dW[i][q].v), I).v);
        const Frag<T> t1 = to_frag<T>(transpose16(to_frag<T>(dW[i][q + 1].v), I).v);
        mma32(t.v, eGF[0][q], eGF[0][q + 1], t0, t1);
      }
      sh.tr[i][l] = t.v;
    }
  }

  // dW += XQ^T dZb + XK^T dZ1 ; db += colsum(dZb + dZ1)
  __device__ void accumulate(int s) {
    const int par = s & 1;
    Frag<T> xqTf[FT], xkTf[FT], dzbf[FT], dz1f[FT];
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      xqTf[q] = sh.xq[par][q][l];
      xkTf[q] = sh.xk[par][q][l];
      dzbf[q] = sh.dzb[par][q][l];
      dz1f[q] = sh.dz1[q][l];
    }
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) mma32(dW[i][o].v, xqTf[i], xkTf[i], dzbf[o], dz1f[o]);
#pragma unroll
    for (int o = 0; o < FT; ++o) db_tm[o] += sh.db[16 * o + n];
  }

  __device__ void finish() {
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) store_tile(p.dW + (size_t)c.chain * F * F, F, 16 * i, 16 * o, dW[i][o]);
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < FT; ++o) p.db[(size_t)c.chain * F + 16 * o + n] = db_tm[o];
    }
  }
};

template <typename T, int FT>
__global__ __launch_bounds__(128) void linear_bwd_kernel(LinearBwdParams p) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  __shared__ LinBwdShared<T, FT> sh;
  LinBwdCtx<T, FT> c;
  c.chain = blockIdx.x;
  c.h = c.chain % p.H;
  c.NC = p.NC;
  c.G = p.G;
  c.NK = p.NK;
  const size_t xoff = (size_t)c.chain * c.NC * K * F;
  const size_t eoff = (size_t)c.chain * c.NC * K * K;
  c.XQ = static_cast<const T*>(p.XQ) + xoff;
  c.XK = static_cast<const T*>(p.XK) + xoff;
  c.XV = static_cast<const T*>(p.XV) + xoff;
  c.DO = static_cast<const T*>(p.dout) + xoff;
  c.ETA = static_cast<const T*>(p.eta) + eoff;
  c.DXQ = static_cast<T*>(p.dXQ) + xoff;
  c.DXK = static_cast<T*>(p.dXK) + xoff;
  c.DXV = static_cast<T*>(p.dXV) + xoff;
  c.DETA = static_cast<T*>(p.deta) + eoff;
  c.WS = p.ws + (size_t)c.chain * c.G * K * F;

  // Both waves execute the same sequence of barriers: per group one after
  // phase 1, then two per mini-batch.
  if (threadIdx.x < 64) {
    Wave0<T, FT> w(p, c, sh);
    for (int kk = c.NK - 1; kk >= 0; --kk) {
      const int s0 = kk * c.G, s1 = min(s0 + c.G, c.NC);
      w.recompute_group(kk, s0, s1);
      __syncthreads();
      w.step_a(s1 - 1, s0);
      for (int s = s1 - 1; s >= s0; --s) {
        __syncthreads();  // wave 1 has posted the carry terms of s
        w.step_b(s, s0);
        __syncthreads();  // dZb, dZ1 of s posted
        if (s > s0) w.step_a(s - 1, s0);
      }
    }
    w.finish();
  } else {
    Wave1<T, FT> w(p, c, sh);
    for (int kk = c.NK - 1; kk >= 0; --kk) {
      const int s0 = kk * c.G, s1 = min(s0 + c.G, c.NC);
      __syncthreads();
      for (int s = s1 - 1; s >= s0; --s) {
        w.carry_terms(s, s0);
        __syncthreads();
        __syncthreads();
        w.accumulate(s);
      }
    }
    w.finish();
  }
}

template <typename T, int FT>
static hipError_t launch_bwd(const LinearBwdParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((linear_bwd_kernel<T, FT>), dim3(p.B * p.H), dim3(128), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_linear_bwd(const LinearBwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_bwd<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_bwd<__bf16, 2>(p, stream);
  } else {
    if (p.F == 64) return launch_bwd<float, 4>(p, stream);
    if (p.F == 32) return launch_bwd<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
