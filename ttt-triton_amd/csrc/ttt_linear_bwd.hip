// TTT-Linear backward on gfx950: one workgroup of three wavefronts per
// (batch, head) chain, one reverse sweep over all NC mini-batches.
//
// The forward saves, per mini-batch, the inner-loss gradient G_s, the
// normalised Z1 with its row statistics and the normalised readout Zb with its
// token statistics (LinSavedSlot).  With those the backward needs the fast
// weight only for the products dZb W_s^T and dZ1 W_s^T, and the only
// sequential dependency left is the gradient wrt the state after mini-batch s,
// dW' and db' (ops/ttt_linear.py:8-54 differentiated by hand):
//   dG_s = -M^T dZb - diag(e) (XK dW' + db')      (e = eta[K-1])
//   dZ1  = backward of ln_fused_l2_bwd at dG_s     (dtgt = dXV alongside)
//   dW   = dW' + XQ^T dZb + XK^T dZ1 ;  db = db' + colsum(dZb + dZ1)
// The three waves form a pipeline with one barrier per iteration: in
// iteration it, wave P works on mini-batch NC-1-it, wave S on NC-it and wave X
// on NC+1-it.
//   P (prepare)  everything that involves neither W nor dW: the readout-LN
//                backward (dZb), the dual-form terms (dM, dA, deta),
//                -M^T dZb and the exact transposes the other two waves
//                consume;
//   S (state)    owns dW and db: XK dW' + db', the inner-loss LN backward,
//                the dW/db update, and hands dW' to X as operand frags;
//   X (weights)  owns W^T, rebuilt backwards from the checkpoint after each
//                group (kernels/linear_backward.py:278 walks the same groups):
//                W_s = W_{s+1} + XK_s^T diag(e) G_s with the forward's MFMA
//                operands; forms dXQ, dXK, dXV and deta (with the
//                dual-form terms dout + dA XK and dA^T XQ from P's dA, and
//                -(e G) dW'^T from S's dW') and writes them.
// Feature-major tiles ("FM": lane (g, n) holds features 16o + 4g + j of token
// n) are what the outputs are written from, 4 contiguous elements per lane.
#include "ttt_eta.h"
#include "ttt_kernels.h"
#include "ttt_ln.h"

namespace ttt {

// whether S hands dW' to X as operand frags (16-bit) or forms -(e G) dW'^T itself
template <typename T> constexpr bool kLinHandDw = sizeof(T) == 2;

template <typename T, int FT> struct LinBwdShared {
  // P -> S, by mini-batch parity
  struct PS {
    Frag<T> xk[FT][64];     // XK row-major frags (free = token)
    Frag<T> xq_t[FT][64];   // XQ token-major tiles as frags (free = feature)
    Frag<T> dzb_t[FT][64];  // dZb token-major tiles as frags (free = feature)
    Frag<T> egn[FT][64];    // -(e G) row-major frags (free = token)
    f4 dg0[FT][64];         // -M^T dZb, token-major
    f4 tgt[FT][64];         // XV - XK, token-major
    f4 e[64];               // eta[K-1][4g + j]
    float dbz[16 * FT];     // column sums of dZb
  } ps[2];
  // P -> S and X, by mini-batch mod 3
  struct PX {
    Frag<T> xk_t[FT][64];   // XK token-major tiles as frags (free = feature)
    Frag<T> dzb[FT][64];    // dZb row-major frags (free = token)
    Frag<T> eg_t[FT][64];   // e G token-major tiles as frags (free = feature)
    Frag<T> xq_t[FT][64];   // XQ token-major tiles as frags (free = feature)
    Frag<T> dat[64];        // dA^T [t_k x t_q] as a frag
    Frag<T> egn[kLinHandDw<T> ? FT : 1][64];  // -(e G) row-major frags (free = token), for X (16-bit)
    Frag<T> da[64];         // dA [t_q x t_k] as a frag
    f4 det[64];             // deta without the last-row term: lane (g, n) holds deta[n][4g + j]
  } px[3];
  // S -> X, by mini-batch parity
  struct SX {
    Frag<T> dz1_t[FT][64];   // dZ1 token-major tiles as frags
    Frag<T> dtgt_t[FT][64];  // dtgt (= dXV) token-major tiles as frags
    // 16-bit: dW' (not yet updated) as operand frags, dwf[i][o] of block (i, o),
    // for X to form (-(e G) dW'^T)^T; fp32 (twice the bytes, beyond the LDS):
    // S forms it, FM
    Frag<T> dwf[kLinHandDw<T> ? FT : 1][kLinHandDw<T> ? FT : 1][64];
    f4 tr[kLinHandDw<T> ? 1 : FT][64];
    f4 de[64];               // last-row eta gradient of token 4g + j
  } sx[2];
  float red[2 * 16 * FT];    // readout-LN parameter gradients, P -> S at the end
};

template <typename T, int FT> struct LinBwdCtx {
  const T *XQ, *XK, *XV, *DO;
  T *DXQ, *DXK, *DXV;
  const void* ETA;   // dense eta [NC][K][K] and its gradient, in the kernel's eta type
  void* DETA;
  const float* LRP;  // lr [NC][K] when eta is given as learning rates
  float* DLR;        // dlr [NC][K] then
  int eta_rule;
  const char* SV;  // this chain's saved slots
  int NC, G, NK, chain, h;
};

// ------------------------------------------------------------------ wave P
template <typename T, int FT, bool LR, typename ET> struct WaveP {
  static constexpr int F = 16 * FT;
  static constexpr int K = 16;
  using Slot = LinSavedSlot<F>;
  const LinBwdCtx<T, FT>& c;
  LinBwdShared<T, FT>& sh;
  int l, g, n;
  Frag<T> I;
  f4 lnw_fm[FT];
  f4 aw[FT], ab[FT];  // readout-LN parameter gradient partials (features 16o + 4g + j, tokens of this lane)
  struct In {
    Frag<T> xq[1][FT], xk[1][FT], xv[FT], dof[FT];
    Frag<ET> etaT, e;  // raw: converted where used, so the prefetch is not waited for
    f4 etan;           // fp32 eta under 16-bit activations: eta[4g + j][n], read as it is
    f4 lr4;           // LR: lr[4g .. 4g+3] and lr[n], expanded where used
    float lrn;
    f4 G[FT], xhb[FT];
    float rsb;
  } in;

  __device__ WaveP(const LinearBwdParams& p, const LinBwdCtx<T, FT>& c_, LinBwdShared<T, FT>& sh_) : c(c_), sh(sh_) {
    l = lane_id();
    g = l >> 4;
    n = l & 15;
    I = identity_frag<T>();
#pragma unroll
    for (int o = 0; o < FT; ++o) {
#pragma unroll
      for (int j = 0; j < 4; ++j) lnw_fm[o][j] = p.ln_w[c.h * F + 16 * o + 4 * g + j];
      aw[o] = f4{0.f, 0.f, 0.f, 0.f};
      ab[o] = f4{0.f, 0.f, 0.f, 0.f};
    }
  }

  __device__ void load(int s) {
    const size_t xo = (size_t)s * K * F;
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      in.xq[0][q] = load_frag(c.XQ + xo, F, 16 * q);
      in.xk[0][q] = load_frag(c.XK + xo, F, 16 * q);
      in.xv[q] = load_frag(c.XV + xo, F, 16 * q);
      in.dof[q] = load_frag(c.DO + xo, F, 16 * q);
    }
    if constexpr (LR) {
      in.lr4 = *reinterpret_cast<const f4*>(c.LRP + (size_t)s * K + 4 * g);
      in.lrn = c.LRP[(size_t)s * K + n];
    } else {
      const ET* etas = static_cast<const ET*>(c.ETA) + (size_t)s * K * K;
      in.etaT = load_frag(etas, K, 0);            // lane (g, n): eta[n][4g + j]
      in.e = load_frag(etas + (K - 1) * K, 0, 0);  // eta[K-1][4g + j]
      if constexpr (sizeof(ET) != sizeof(T)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) in.etan[j] = etas[(4 * g + j) * K + n];
      }
    }
    const float* sv = reinterpret_cast<const float*>(c.SV + (size_t)s * Slot::BYTES);
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      in.G[o] = fill_tile(sv + Slot::G / 4 + o * 256).v;
      in.xhb[o] = fill_tile(sv + Slot::XHB / 4 + o * 256).v;
    }
    in.rsb = sv[Slot::RSB / 4 + n];
  }

  __device__ void step(int s, int m3) {
    const In x = in;
    load(s > 0 ? s - 1 : 0);  // unconditional, so that the wait for it is exact
    auto& ps = sh.ps[s & 1];
    auto& px = sh.px[m3];
    const f4 etaT = LR ? eta_rowfrag_from_lr(c.eta_rule, x.lr4) : frag_to_f4(x.etaT);
    const f4 e = LR ? eta_lastrow_from_lr(x.lr4) : frag_to_f4(x.e);

    Frag<T> xqTf[FT], xkTf[FT];
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      const Tile xkT = transpose16(x.xk[0][q], I);
      xkTf[q] = to_frag<T>(xkT.v);
      xqTf[q] = to_frag<T>(transpose16(x.xq[0][q], I).v);
      ps.tgt[q][l] = transpose16(x.xv[q], I).v - xkT.v;
      ps.xk[q][l] = x.xk[0][q];
      ps.xq_t[q][l] = xqTf[q];
      px.xq_t[q][l] = xqTf[q];
      px.xk_t[q][l] = xkTf[q];
    }
    ps.e[l] = e;

    // e G (the forward's update operand with the sign flipped), -(e G) and G
    // as row-major frags
    Frag<T> GF[1][FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      f4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = e[j] * x.G[o][j];
      const Frag<T> ge = to_frag<T>(v);
      px.eg_t[o][l] = ge;
      const Frag<T> egn = negate(to_frag<T>(transpose16(ge, I).v));
      ps.egn[o][l] = egn;
      if constexpr (kLinHandDw<T>) px.egn[o][l] = egn;
      GF[0][o] = to_frag<T>(transpose16(to_frag<T>(x.G[o]), I).v);
    }

    // A^T = XK XQ^T [t_k x t_q], A = XQ XK^T [t_q x t_k]; M = eta (.) A + eta
    Tile at[1][1], a[1][1];
    at[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
    a[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
    gemm<1, 1, FT>(at, x.xk, x.xq);
    gemm<1, 1, FT>(a, x.xq, x.xk);
    // lane (g, n): eta[4g + j][n]
    f4 eta_n;
    if constexpr (LR)
      eta_n = eta_ctile_from_lr(c.eta_rule, x.lrn);
    else if constexpr (sizeof(ET) != sizeof(T))
      eta_n = x.etan;  // (the identity product runs on T's matrix cores)
    else
      eta_n = transpose16(x.etaT, I).v;
    f4 m;
#pragma unroll
    for (int j = 0; j < 4; ++j) m[j] = eta_n[j] * a[0][0].v[j] + eta_n[j];

    // readout LayerNorm backward (FM)
    Frag<T> dZbF[1][FT], dZbTf[FT];
    {
      constexpr float invF = 1.0f / F;
      f4 gy[FT];
      float a1 = 0.f, a2 = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const f4 d = frag_to_f4(x.dof[o]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          gy[o][j] = d[j] * lnw_fm[o][j];
          aw[o][j] += d[j] * x.xhb[o][j];
          ab[o][j] += d[j];
          a1 += gy[o][j];
          a2 += gy[o][j] * x.xhb[o][j];
        }
      }
      a1 = sum_col4(a1) * invF;
      a2 = sum_col4(a2) * invF;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        f4 dz;
#pragma unroll
        for (int j = 0; j < 4; ++j) dz[j] = x.rsb * (gy[o][j] - a1 - x.xhb[o][j] * a2);
        dZbF[0][o] = to_frag<T>(dz);
        px.dzb[o][l] = dZbF[0][o];
        dZbTf[o] = to_frag<T>(transpose16(dZbF[0][o], I).v);
        ps.dzb_t[o][l] = dZbTf[o];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float cs = sum_row16(dz[j]);
          if (n == 0) ps.dbz[16 * o + 4 * g + j] = cs;
        }
      }
    }

    // dM = -dZb G^T; dA = dM (.) eta; deta = dM (.) (A + 1) (+ the last-row term in S)
    Tile dm[1][1], dmT[1][1];
    dm[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
    dmT[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
    gemm<1, 1, FT>(dm, dZbF, GF);   // dZb G^T  [t_q x t_k]
    gemm<1, 1, FT>(dmT, GF, dZbF);  // G dZb^T  [t_k x t_q]
    f4 det, daT, da;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      det[j] = -dmT[0][0].v[j] * (1.0f + at[0][0].v[j]);
      daT[j] = -dmT[0][0].v[j] * etaT[j];
      da[j] = -dm[0][0].v[j] * eta_n[j];
    }
    px.det[l] = det;
    const Frag<T> daTf = to_frag<T>(daT), daf = to_frag<T>(da), mf = to_frag<T>(-m);
    px.dat[l] = daTf;  // (dout + dA XK)^T and (dA^T XQ)^T are formed by X
    px.da[l] = daf;
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      f4 dg = f4{0.f, 0.f, 0.f, 0.f};
      mma16(dg, mf, dZbTf[q]);  // -M^T dZb
      ps.dg0[q][l] = dg;
    }
  }

  // readout-LN parameter gradients summed over the chain's tokens
  __device__ void finish() {
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float w = sum_row16(aw[o][j]);
        const float b = sum_row16(ab[o][j]);
        if (n == 0) {
          sh.red[16 * o + 4 * g + j] = w;
          sh.red[F + 16 * o + 4 * g + j] = b;
        }
      }
  }
};

// ------------------------------------------------------------------ wave S
template <typename T, int FT> struct WaveS {
  static constexpr int F = 16 * FT;
  static constexpr int K = 16;
  using Slot = LinSavedSlot<F>;
  const LinBwdCtx<T, FT>& c;
  LinBwdShared<T, FT>& sh;
  int l, g, n;
  Frag<T> I;
  float lnw_tm[FT], lnb_tm[FT];
  float dlnw_tm[FT], dlnb_tm[FT];
  Tile dW[FT][FT];
  float db_tm[FT];
  struct In {
    f4 G[FT], xh[FT];
    f4 rstd, cc;
  } in;

  __device__ WaveS(const LinearBwdParams& p, const LinBwdCtx<T, FT>& c_, LinBwdShared<T, FT>& sh_) : c(c_), sh(sh_) {
    l = lane_id();
    g = l >> 4;
    n = l & 15;
    I = identity_frag<T>();
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      lnw_tm[o] = p.ln_w[c.h * F + 16 * o + n];
      lnb_tm[o] = p.ln_b[c.h * F + 16 * o + n];
      dlnw_tm[o] = 0.f;
      dlnb_tm[o] = 0.f;
      db_tm[o] = 0.f;
#pragma unroll
      for (int i = 0; i < FT; ++i) dW[i][o].v = f4{0.f, 0.f, 0.f, 0.f};
    }
  }

  __device__ void load(int s) {
    const float* sv = reinterpret_cast<const float*>(c.SV + (size_t)s * Slot::BYTES);
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      in.G[o] = fill_tile(sv + Slot::G / 4 + o * 256).v;
      in.xh[o] = fill_tile(sv + Slot::XH / 4 + o * 256).v;
    }
    in.rstd = load4(sv + Slot::RSTD / 4 + 4 * g);
    in.cc = load4(sv + Slot::CC / 4 + 4 * g);
  }

  __device__ void step(int s, int m3) {
    const In x = in;
    load(s > 0 ? s - 1 : 0);  // unconditional, so that the wait for it is exact
    const auto& ps = sh.ps[s & 1];
    const auto& px = sh.px[m3];
    auto& sx = sh.sx[s & 1];

    // XK dW' + db'
    Frag<T> xk[1][FT];
#pragma unroll
    for (int q = 0; q < FT; ++q) xk[0][q] = ps.xk[q][l];
    Tile qm[1][FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) qm[0][o].v = f4{db_tm[o], db_tm[o], db_tm[o], db_tm[o]};
    gemm_pt<1, FT, FT>(qm, xk, dW);

    // dG = -M^T dZb - e (XK dW' + db');  de = -rowsum(G (XK dW' + db'))
    const f4 e = ps.e[l];
    Tile dG[FT], Gt[FT];
    f4 dep = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      const f4 d0 = ps.dg0[o][l];
      Gt[o].v = x.G[o];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dG[o].v[j] = d0[j] - e[j] * qm[0][o].v[j];
        dep[j] += x.G[o][j] * qm[0][o].v[j];
      }
    }
    {
      f4 de;
#pragma unroll
      for (int j = 0; j < 4; ++j) de[j] = -sum_row16(dep[j]);
      sx.de[l] = de;
    }

    if constexpr (kLinHandDw<T>) {
      // dW' as operand frags for X, which forms (-(e G) dW'^T)^T
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) sx.dwf[i][o][l] = to_frag<T>(dW[i][o].v);
    } else {
      // (-(e G) dW'^T)^T from the transposed dW' blocks (FM)
      Frag<T> egn[FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) egn[o] = ps.egn[o][l];
#pragma unroll
      for (int i = 0; i < FT; ++i) {
        f4 t = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < FT; o += 2) {
          const Frag<T> t0 = to_frag<T>(transpose16(to_frag<T>(dW[i][o].v), I).v);
          const Frag<T> t1 = to_frag<T>(transpose16(to_frag<T>(dW[i][o + 1].v), I).v);
          mma32(t, t0, t1, egn[o], egn[o + 1]);
        }
        sx.tr[i][l] = t;
      }
    }

    // backward of the inner-loss LayerNorm
    LnL2Lite<FT> ln;
    ln.rstd = x.rstd;
    ln.c = x.cc;
    f4 tgt[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      ln.xh[o] = x.xh[o];
      tgt[o] = ps.tgt[o][l];
    }
    f4 dz1[FT], dtgt[FT];
    ln.backward(dG, Gt, tgt, lnw_tm, lnb_tm, dz1, dtgt, dlnw_tm, dlnb_tm);

    // dW += XQ^T dZb + XK^T dZ1 ;  db += colsum(dZb + dZ1)
    Frag<T> dz1f[FT], dzbf[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      dz1f[o] = to_frag<T>(dz1[o]);
      dzbf[o] = ps.dzb_t[o][l];
      sx.dz1_t[o][l] = dz1f[o];
      sx.dtgt_t[o][l] = to_frag<T>(dtgt[o]);
    }
#pragma unroll
    for (int i = 0; i < FT; ++i) {
      const Frag<T> xqTf = ps.xq_t[i][l], xkTf = px.xk_t[i][l];
#pragma unroll
      for (int o = 0; o < FT; ++o) mma32(dW[i][o].v, xqTf, xkTf, dzbf[o], dz1f[o]);
    }
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc += dz1[o][j];
      db_tm[o] += sum_col4(acc) + ps.dbz[16 * o + n];
    }
  }

  __device__ void finish(const LinearBwdParams& p) {
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) store_tile(p.dW + (size_t)c.chain * F * F, F, 16 * i, 16 * o, dW[i][o]);
    float lw_t[FT], lb_t[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      lw_t[o] = sum_col4(dlnw_tm[o]);
      lb_t[o] = sum_col4(dlnb_tm[o]);
    }
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        p.db[(size_t)c.chain * F + 16 * o + n] = db_tm[o];
        p.dln_w[(size_t)c.chain * F + 16 * o + n] = lw_t[o] + sh.red[16 * o + n];
        p.dln_b[(size_t)c.chain * F + 16 * o + n] = lb_t[o] + sh.red[F + 16 * o + n];
      }
    }
  }
};

// ------------------------------------------------------------------ wave X
template <typename T, int FT, bool LR, typename ET> struct WaveX {
  static constexpr int F = 16 * FT;
  static constexpr int K = 16;
  const LinearBwdParams& p;
  const LinBwdCtx<T, FT>& c;
  LinBwdShared<T, FT>& sh;
  int l, g, n;
  Frag<T> I;
  Tile WT[FT][FT];  // WT[o][i]: lane (g, n) holds W[16i + n][16o + 4g + j]
  Tile WN[FT][FT];  // the checkpoint the next group starts from
  Frag<T> dof_n[FT];  // dout of the next mini-batch (FM)

  __device__ WaveX(const LinearBwdParams& p_, const LinBwdCtx<T, FT>& c_, LinBwdShared<T, FT>& sh_)
      : p(p_), c(c_), sh(sh_) {
    l = lane_id();
    g = l >> 4;
    n = l & 15;
    I = identity_frag<T>();
  }

  __device__ void load_do(int s) {
#pragma unroll
    for (int q = 0; q < FT; ++q) dof_n[q] = load_frag(c.DO + (size_t)s * K * F, F, 16 * q);
  }

  __device__ void load_w(Tile (&w)[FT][FT], const float* src) {
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int i = 0; i < FT; ++i) w[o][i].v = load4(src + (16 * i + n) * F + 16 * o + 4 * g);
  }

  __device__ void step(int s, int m3) {
    // W entering step s+1: the final state, or the checkpoint prefetched in
    // the previous step, at the end of each group
    if (s + 1 < c.NC && (s + 1) % c.G == 0) {
#pragma unroll
      for (int o = 0; o < FT; ++o)
#pragma unroll
        for (int i = 0; i < FT; ++i) WT[o][i] = WN[o][i];
    }
    // prefetch the checkpoint entering this group when s starts one
    if (s > 0 && s % c.G == 0) load_w(WN, p.W_ckpt + ((size_t)c.chain * c.NK + s / c.G) * F * F);

    const auto& px = sh.px[m3];
    const auto& sx = sh.sx[s & 1];
    Frag<T> dof[FT];
#pragma unroll
    for (int q = 0; q < FT; ++q) dof[q] = dof_n[q];
    load_do(s > 0 ? s - 1 : 0);  // unconditional, so that the wait for it is exact
    // W_s = W_{s+1} + XK^T diag(e) G:  W^T[o][i] += sum_t (e G)[t][o] XK[t][i]
    {
      Frag<T> xkTf[FT];
#pragma unroll
      for (int i = 0; i < FT; ++i) xkTf[i] = px.xk_t[i][l];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const Frag<T> ge = px.eg_t[o][l];
#pragma unroll
        for (int i = 0; i < FT; ++i) mma16(WT[o][i].v, ge, xkTf[i]);
      }
    }

    // dXQ^T = (dout + dA XK)^T + W dZb^T
    // dXK^T = (dA^T XQ)^T - dtgt^T + (-(e G) dW'^T)^T + W dZ1^T
    Frag<T> dzbF[FT], dz1F[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      dzbF[o] = px.dzb[o][l];
      dz1F[o] = to_frag<T>(transpose16(sx.dz1_t[o][l], I).v);
    }
    const size_t xo = (size_t)s * K * F;
    const Frag<T> daTf = px.dat[l], daf = px.da[l];
#pragma unroll
    for (int i = 0; i < FT; ++i) {
      const f4 dv = transpose16(sx.dtgt_t[i][l], I).v;
      f4 q = frag_to_f4(dof[i]);
      mma16(q, px.xk_t[i][l], daTf);  // + (dA XK)^T
      f4 xkp = f4{0.f, 0.f, 0.f, 0.f};
      mma16(xkp, px.xq_t[i][l], daf);  // (dA^T XQ)^T
      // (-(e G) dW'^T)^T from the transposed dW' blocks (FM)
      f4 tr;
      if constexpr (kLinHandDw<T>) {
        tr = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < FT; o += 2) {
          const Frag<T> t0 = to_frag<T>(transpose16(sx.dwf[i][o][l], I).v);
          const Frag<T> t1 = to_frag<T>(transpose16(sx.dwf[i][o + 1][l], I).v);
          mma32(tr, t0, t1, px.egn[o][l], px.egn[o + 1][l]);
        }
      } else {
        tr = sx.tr[i][l];
      }
      f4 k = xkp + tr - dv;
#pragma unroll
      for (int o = 0; o < FT; o += 2) {
        const Frag<T> w0 = to_frag<T>(WT[o][i].v), w1 = to_frag<T>(WT[o + 1][i].v);
        mma32(q, w0, w1, dzbF[o], dzbF[o + 1]);
        mma32(k, w0, w1, dz1F[o], dz1F[o + 1]);
      }
      store_f4(c.DXQ + xo, F, 16 * i, q);
      store_f4(c.DXK + xo, F, 16 * i, k);
      store_f4(c.DXV + xo, F, 16 * i, dv);
    }
    f4 det = px.det[l];
    if (n == K - 1) det += sx.de[l];
    if constexpr (LR) {
      // dlr of columns 4g..4g+3: the 16 lanes of group g store the same value
      *reinterpret_cast<f4*>(c.DLR + (size_t)s * K + 4 * g) = dlr_from_detaT(c.eta_rule, det);
    } else {
      store_f4(static_cast<ET*>(c.DETA) + (size_t)s * K * K, K, 0, det);
    }
  }
};

template <typename T, int FT, bool LR, typename ET = T>
__global__ __launch_bounds__(192) void linear_bwd_kernel(LinearBwdParams p) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  static_assert(sizeof(LinBwdShared<T, FT>) <= 160 * 1024, "the handoff areas fit one CU's LDS");
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
  c.ETA = LR ? nullptr : static_cast<const ET*>(p.eta) + eoff;
  c.LRP = LR ? static_cast<const float*>(p.eta) + (size_t)c.chain * c.NC * K : nullptr;
  c.DLR = LR ? static_cast<float*>(p.deta) + (size_t)c.chain * c.NC * K : nullptr;
  c.eta_rule = p.eta_rule;
  c.DXQ = static_cast<T*>(p.dXQ) + xoff;
  c.DXK = static_cast<T*>(p.dXK) + xoff;
  c.DXV = static_cast<T*>(p.dXV) + xoff;
  c.DETA = LR ? nullptr : static_cast<ET*>(p.deta) + eoff;
  c.SV = static_cast<const char*>(p.saved) + (size_t)c.chain * c.NC * LinSavedSlot<F>::BYTES;

  // Every wave passes NC + 3 barriers: one per pipeline iteration, one before
  // the final reductions.  Each wave retires its first loads before its loop:
  // loads still pending on loop entry make the wait-count pass wait for every
  // outstanding access in each iteration.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int NC = c.NC;
  if (wave == 0) {
    WaveP<T, FT, LR, ET> w(p, c, sh);
    w.load(NC - 1);
    __builtin_amdgcn_s_waitcnt(0);
    for (int it = 0; it < NC + 2; ++it) {
      const int s = NC - 1 - it;
      if (s >= 0) w.step(s, s % 3);
      __syncthreads();
    }
    w.finish();
    __syncthreads();
  } else if (wave == 1) {
    WaveS<T, FT> w(p, c, sh);
    w.load(NC - 1);
    __builtin_amdgcn_s_waitcnt(0);
    for (int it = 0; it < NC + 2; ++it) {
      const int s = NC - it;
      if (s >= 0 && s < NC) w.step(s, s % 3);
      __syncthreads();
    }
    __syncthreads();
    w.finish(p);
  } else {
    WaveX<T, FT, LR, ET> w(p, c, sh);
    w.load_w(w.WT, p.W_last + (size_t)c.chain * F * F);
    w.load_do(NC - 1);
    __builtin_amdgcn_s_waitcnt(0);
    for (int it = 0; it < NC + 2; ++it) {
      const int s = NC + 1 - it;
      if (s >= 0 && s < NC) w.step(s, s % 3);
      __syncthreads();
    }
    __syncthreads();
  }
}

template <typename T, int FT>
static hipError_t launch_bwd(const LinearBwdParams& p, hipStream_t stream) {
  if (p.eta_rule == TTT_ETA_DENSE)
    hipLaunchKernelGGL((linear_bwd_kernel<T, FT, false>), dim3(p.B * p.H), dim3(192), 0, stream, p);
  else if (p.eta_rule == TTT_ETA_DENSE_F32)
    hipLaunchKernelGGL((linear_bwd_kernel<T, FT, false, float>), dim3(p.B * p.H), dim3(192), 0, stream, p);
  else
    hipLaunchKernelGGL((linear_bwd_kernel<T, FT, true>), dim3(p.B * p.H), dim3(192), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_linear_bwd(const LinearBwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_bwd<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_bwd<__bf16, 2>(p, stream);
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_bwd<_Float16, 4>(p, stream);
    if (p.F == 32) return launch_bwd<_Float16, 2>(p, stream);
  } else {
    if (p.F == 64) return launch_bwd<float, 4>(p, stream);
    if (p.F == 32) return launch_bwd<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

size_t linear_saved_slot_bytes(int F) { return lin_saved_slot_bytes(F); }

}  // namespace ttt
