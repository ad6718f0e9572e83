// TTT-MLP mini-batch forward on gfx950.
//
// One workgroup per (batch, head) chain with NW wavefronts of HT hidden tiles
// each (FF = 16 HT NW): at F = 64 always four waves (HT = FF/64), so that the
// LayerNorms split by rows as below; at F = 32 waves of four tiles.  Wave w owns hidden units [16 HT w, 16 HT (w+1)): its
// slice of W1 (F x 16HT) and W2 (16HT x F) stays in registers (fp32, MFMA
// accumulator layout) for all NC mini-batches; b2 is replicated in every wave.  Per mini-batch of K = 16 tokens
// (ops/ttt_mlp.py:9-67, dual form with a full KxK eta):
//
//   Z1 = XK W1 + b1, X2 = gelu(Z1)               per wave, its 64 hidden units
//   Z2 = sum_w X2_w W2_w + b2                     partial sums reduced through LDS
//   G2 = ln_fused_l2_bwd(Z2, XV - XK)             every wave, token-major rows
//   G1 = (G2 W2^T) (.) gelu'(Z1)                  per wave
//   Z1b = XQ W1 - (eta o XQ XK^T + eta) G1 + b1, X2b = gelu(Z1b)
//   Z2b = sum_w X2b_w W2_w - (eta o X2b X2^T + eta) G2 + b2
//   out = XQ + LN(Z2b)                            wave w writes feature tiles w, w+NW, ...
//                                                 (token rows 4w..4w+3 when split by rows)
//   W1 -= XK^T diag(e) G1, W2 -= X2^T diag(e) G2, b -= G^T e   (e = eta[K-1])
//
// Checkpoints hold the state entering mini-batch k*G
// (kernels/mlp_forward.py:84-117); memo snapshot s holds the state after
// mini-batch s*M is applied (kernels/mlp_forward.py:193-226).  When `saved`
// is given, every mini-batch's update operands -e*G1, -e*G2 and bias
// decrements, and the activations its backward needs (gelu(Z1) and its first
// two derivatives folded with G2 W2^T, gelu(Z1b) and its derivative, G2, the
// two LayerNorms' normalised rows and statistics, X2b X2^T) are written
// there (MlpSavedSlot layout): the backward rebuilds the state in reverse
// from the update operands and never re-runs the forward.
//
// eta is read per mini-batch either as the dense [K x K] block or, with LR,
// as the K learning rates that the eta rule expands on chip (ttt_eta.h).
//
// Slabs are read through buffer resources; the next mini-batch's XQ and XK
// are requested right after the first barrier of the current one, before its
// stores (gfx9 retires loads and stores in issue order), so they arrive while
// the rest of the mini-batch computes.
#include "ttt_buf.h"
#include "ttt_eta.h"
#include "ttt_kernels.h"
#include "ttt_ln.h"

namespace ttt {

size_t mlp_saved_slot_bytes(int F, int FF, int dtype) {
  return mlp_saved_slot_bytes_of(F, FF, dtype == TTT_DTYPE_F32 ? 4 : 2);
}

template <int FT, int NW> struct MlpFwdShared {
  f4 z2p[NW][FT][64];   // per-wave partial Z2 (token-major tiles, register order)
  f4 z2bp[NW][FT][64];  // per-wave partial X2b W2
  f4 a2p[NW][64];       // per-wave partial (X2b X2^T)^T
  f4 g2[FT][64];        // G2 (token-major tiles, register order), rows split over the waves
};

// The inner-loss LayerNorm is split over the waves by token rows when there
// are as many waves as 16-feature tiles and F = 64: wave w takes rows
// 4w..4w+3 (lane group g = w of every token-major tile) with lane l on
// feature l, so a row's reductions span the 64 lanes and each lane does 4
// rows instead of 16; G2 is then exchanged through LDS.  The readout's output
// LayerNorm is split the same way: each wave folds its share of the
// -(eta o A2 + eta) G2 term into its partial X2b W2 before the exchange, so
// the four partials of a row add up to Z2b and no wave forms all of it.
template <int FT, int NW> constexpr bool kLnRowSplit = (NW == 4 && FT == 4);

template <typename T, int FT, int NW, int HT, bool LR, typename ET = T>
__global__ __launch_bounds__(64 * NW) void mlp_fwd_kernel(MlpFwdParams p) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  constexpr int FF = 16 * HT * NW;  // HT hidden tiles per wave
  constexpr int ST = (int)sizeof(T);
  constexpr int SE = (int)sizeof(ET);  // dense eta element
  using Slot = MlpSavedSlot<F, FF, ST>;
  __shared__ MlpFwdShared<FT, NW> sh;

  const int chain = blockIdx.x;
  const int h = chain % p.H;
  const int NC = p.NC;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform
  const int l = lane_id(), g = l >> 4, n = l & 15;
  const int hs = 16 * HT * wave;  // first hidden unit of this wave

  // per-chain slabs as buffer resources; lane offsets shared by all of them
  const size_t xoff = (size_t)chain * NC * K * F;
  const size_t eoff = (size_t)chain * NC * K * K;
  const unsigned xbytes = (unsigned)((size_t)NC * K * F * ST), ebytes = (unsigned)((size_t)NC * K * K * SE);
  const rsrc_t rXQ = make_rsrc(static_cast<const T*>(p.XQ) + xoff, xbytes);
  const rsrc_t rXK = make_rsrc(static_cast<const T*>(p.XK) + xoff, xbytes);
  const rsrc_t rXV = make_rsrc(static_cast<const T*>(p.XV) + xoff, xbytes);
  const rsrc_t rET = LR ? make_rsrc(static_cast<const float*>(p.eta) + (size_t)chain * NC * K, NC * K * 4)
                        : make_rsrc(static_cast<const ET*>(p.eta) + eoff, ebytes);
  const int eta_rule = p.eta_rule;
  const rsrc_t rOUT = make_rsrc(static_cast<T*>(p.out) + xoff, xbytes);
  const int xl = (n * F + 4 * g) * ST;        // frag lane offset in a [16 x F] block
  const int el = (n * K + 4 * g) * SE;        // frag lane offset in a [16 x 16] eta block
  const int e4 = ((K - 1) * K + 4 * g) * SE;  // eta[K-1][4g .. 4g+3]
  const int w1l = ((4 * g) * FF + hs + n) * 4;  // [F][FF] tile lane offset, columns hs + ...
  const int w2l = ((hs + 4 * g) * F + n) * 4;   // [FF][F] tile lane offset, rows hs + ...
  const bool want_saved = p.saved != nullptr;
  const rsrc_t rSV = make_rsrc(want_saved ? static_cast<char*>(p.saved) + (size_t)chain * NC * Slot::BYTES : nullptr,
                               want_saved ? (unsigned)(NC * Slot::BYTES) : 0u);
  const int g1l = ((wave * HT) * 64 + l) * 4 * ST;  // + o * 256 * ST: this wave's [16 x 64] slice, lane order
  const int g2l = l * 4 * ST;                       // + c * 256 * ST: [16 x F], lane order
  const int f4l = l * 16;                           // + c * 1024: fp32 tiles, lane order
  const int a2l = (4 * g * 16 + n) * 4;             // C-layout tile of a row-major [16 x 16] fp32 block

  // state slice: W1[:, hs:hs+64] as tiles [f block][hidden block], W2[hs:hs+64, :]
  Tile W1[FT][HT], W2[HT][FT];
  float b1_tm[HT], b2_tm[FT];
  {
    const rsrc_t r1 = make_rsrc(p.W1_init + (size_t)chain * F * FF, F * FF * 4);
    const rsrc_t r2 = make_rsrc(p.W2_init + (size_t)chain * FF * F, FF * F * 4);
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) W1[i][o] = bload_tile(r1, w1l, 0, FF, 16 * i, 16 * o);
#pragma unroll
    for (int i = 0; i < HT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) W2[i][o] = bload_tile(r2, w2l, 0, F, 16 * i, 16 * o);
#pragma unroll
    for (int o = 0; o < HT; ++o) b1_tm[o] = p.b1_init[(size_t)chain * FF + hs + 16 * o + n];
#pragma unroll
    for (int o = 0; o < FT; ++o) b2_tm[o] = p.b2_init[(size_t)chain * F + 16 * o + n];
  }
  float lnw_tm[FT], lnb_tm[FT];
#pragma unroll
  for (int o = 0; o < FT; ++o) {
    lnw_tm[o] = p.ln_w[h * F + 16 * o + n];
    lnb_tm[o] = p.ln_b[h * F + 16 * o + n];
  }
  const float lnw_l = kLnRowSplit<FT, NW> ? p.ln_w[h * F + l] : 0.f;  // feature l (row-split LayerNorm)
  const float lnb_l = kLnRowSplit<FT, NW> ? p.ln_b[h * F + l] : 0.f;
  // feature 16 wave + n: the readout's output tile of this wave when NW == FT
  const float lnw_own = NW == FT ? p.ln_w[h * F + 16 * wave + n] : 0.f;
  const float lnb_own = NW == FT ? p.ln_b[h * F + 16 * wave + n] : 0.f;
  const float eps = p.eps;
  const Frag<T> I = identity_frag<T>();

  // writes the state to its non-null destinations; W1's tiles are first
  // transposed exactly (fp32 MFMA against the identity) into row order, so
  // each lane stores 4 consecutive floats of one row with one 16-byte store
  auto store_state = [&](float* w1d, float* b1d, float* w2d, float* b2d) {
    const rsrc_t r1 = make_rsrc(w1d, F * FF * 4);
    const Frag<float> I32 = identity_frag<float>();
    const int w1r = (n * FF + hs + 4 * g) * 4;  // row n, columns hs + 4g .. +3 of a tile
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o)
        bstore_frag<float>(r1, w1r, (16 * i * FF + 16 * o) * 4, Frag<float>{transpose16(Frag<float>{W1[i][o].v}, I32).v});
    if (w2d != nullptr) {
      const rsrc_t r2 = make_rsrc(w2d, FF * F * 4);
#pragma unroll
      for (int i = 0; i < HT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) bstore_tile(r2, w2l, 0, F, 16 * i, 16 * o, W2[i][o]);
    }
    if (g == 0 && b1d != nullptr) {
#pragma unroll
      for (int o = 0; o < HT; ++o) b1d[hs + 16 * o + n] = b1_tm[o];
    }
    if (g == 0 && wave == 0 && b2d != nullptr) {
#pragma unroll
      for (int o = 0; o < FT; ++o) b2d[16 * o + n] = b2_tm[o];
    }
  };

  // XQ, XK of the current mini-batch (frags: free = token, k = feature)
  Frag<T> xq[1][FT], xk[1][FT];
#pragma unroll
  for (int q = 0; q < FT; ++q) {
    xq[0][q] = bload_frag<T>(rXQ, xl + 16 * q * ST, 0);
    xk[0][q] = bload_frag<T>(rXK, xl + 16 * q * ST, 0);
  }
  // retire the loads issued so far: pending on loop entry, they make the
  // wait-count pass wait for every outstanding access in each iteration
  __builtin_amdgcn_s_waitcnt(0);

  for (int s = 0; s < NC; ++s) {
    // the state stays in the accumulator registers (the MFMA update's own),
    // not copied out to VGPRs and back around the phases that read it
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) asm volatile("" : "+a"(W1[i][o].v));
#pragma unroll
    for (int i = 0; i < HT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) asm volatile("" : "+a"(W2[i][o].v));
    if (p.W1_ckpt != nullptr && (s % p.G) == 0) {
      const size_t k = (size_t)chain * p.NK + s / p.G;
      store_state(p.W1_ckpt + k * F * FF, p.b1_ckpt ? p.b1_ckpt + k * FF : nullptr,
                  p.W2_ckpt ? p.W2_ckpt + k * FF * F : nullptr, p.b2_ckpt ? p.b2_ckpt + k * F : nullptr);
    }
    const int xo = s * K * F * ST, eo = s * K * K * SE;
    const int us = s * Slot::BYTES;
    // the inner loss's target XV - XK: as frags (free = token), or, split by
    // rows, rows 4*wave+j of feature l (and XQ's for the output's residual)
    Frag<T> xv[FT], xvr, xkr, xqr;
    if constexpr (kLnRowSplit<FT, NW>) {
      xvr = bload_ctile<T>(rXV, l * ST, xo + 4 * wave * F * ST, F);
      xkr = bload_ctile<T>(rXK, l * ST, xo + 4 * wave * F * ST, F);
      xqr = bload_ctile<T>(rXQ, l * ST, xo + 4 * wave * F * ST, F);
    } else {
#pragma unroll
      for (int q = 0; q < FT; ++q) xv[q] = bload_frag<T>(rXV, xl + 16 * q * ST, xo);
    }
    // dense: eta[n][4g+j] ([t_k x t_q]) and the last eta row; LR: lr[4g .. 4g+3]
    Frag<ET> etaTf, ef;
    f4 lr4;
    if constexpr (LR) {
      lr4 = bload_frag<float>(rET, 16 * g, s * K * 4).v;
    } else {
      etaTf = bload_frag<ET>(rET, el, eo);
      ef = bload_frag<ET>(rET, e4, eo);
    }

    // ---- layer 1 on this wave's hidden units (token-major)
    Frag<T> x2f[HT];     // token-major frags of X2 (free = hidden, k = t)
    Frag<T> x2F[1][HT];  // feature-major frags of X2 (free = t, k = hidden)
    f4 gp[HT];           // gelu'(Z1)
    f4 gpp[HT];          // gelu''(Z1)
    {
      Tile z1[1][HT];
#pragma unroll
      for (int o = 0; o < HT; ++o) z1[0][o].v = f4{b1_tm[o], b1_tm[o], b1_tm[o], b1_tm[o]};
      gemm_pt<1, HT, FT>(z1, xk, W1);
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        f4 x2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float y, dy, ddy;
          gelu_all(z1[0][o].v[j], y, dy, ddy);
          x2[j] = y;
          gp[o][j] = dy;
          gpp[o][j] = ddy;
        }
        bstore_frag<T>(rSV, g1l + o * 256 * ST, us + Slot::SP1, to_frag<T>(gp[o]));
        x2f[o] = to_frag<T>(x2);
        bstore_frag<T>(rSV, g1l + o * 256 * ST, us + Slot::X2, x2f[o]);
        x2F[0][o] = to_frag<T>(transpose16(x2f[o], I).v);
      }
    }
    {
      Tile z2p[1][FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) z2p[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
      gemm_pt<1, FT, HT>(z2p, x2F, W2);
#pragma unroll
      for (int o = 0; o < FT; ++o) sh.z2p[wave][o][l] = z2p[0][o].v;
    }
    __syncthreads();

    // next mini-batch's XQ, XK (the last mini-batch re-reads its own)
    Frag<T> xqn[FT], xkn[FT];
    {
      const int xn = min(s + 1, NC - 1) * K * F * ST;
#pragma unroll
      for (int q = 0; q < FT; ++q) {
        xqn[q] = bload_frag<T>(rXQ, xl + 16 * q * ST, xn);
        xkn[q] = bload_frag<T>(rXK, xl + 16 * q * ST, xn);
      }
    }

    // ---- Z2 and its inner-loss gradient
    Frag<T> xkTf[FT];
    Tile G2[FT];
    if constexpr (kLnRowSplit<FT, NW>) {
#pragma unroll
      for (int q = 0; q < FT; ++q) xkTf[q] = to_frag<T>(transpose16(xk[0][q], I).v);
      // rows 4*wave + j, feature l (= 16 (l >> 4) + n: lane group l >> 4 reads tile l >> 4)
      const int lo = l >> 4;
      const float b2l = lo == 0 ? b2_tm[0] : lo == 1 ? b2_tm[1] : lo == 2 ? b2_tm[2] : b2_tm[3];
      f4 z = f4{b2l, b2l, b2l, b2l};
#pragma unroll
      for (int w = 0; w < NW; ++w) z += sh.z2p[w][lo][16 * wave + n];
      const f4 tgt = frag_to_f4(xvr) - frag_to_f4(xkr);
      constexpr float invF = 1.0f / F;
      f4 rs, xh, gx, g2;
      const f4 mu = sum4_wave(z) * invF;
      const f4 d = z - mu;
      const f4 var = sum4_wave(d * d) * invF;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        rs[j] = rsqrt_f(var[j] + eps);
        xh[j] = d[j] * rs[j];
        gx[j] = (lnw_l * xh[j] + lnb_l - tgt[j]) * lnw_l;
      }
      const f4 s1 = sum4_wave(gx) * invF;
      const f4 cc = sum4_wave(gx * xh) * invF;
#pragma unroll
      for (int j = 0; j < 4; ++j) g2[j] = (gx[j] - s1[j] - xh[j] * cc[j]) * rs[j];
      sh.g2[lo][16 * wave + n] = g2;
      // saved G2, XH (this wave's rows of every tile) and the row statistics
      const int sv = (lo * 64 + 16 * wave + n) * 16;
      bstore_frag<float>(rSV, sv, us + Slot::G2, Frag<float>{g2});
      bstore_frag<float>(rSV, sv, us + Slot::XH, Frag<float>{xh});
      bstore_frag<float>(rSV, keep_or_drop((16 * wave + n) * 16, lo == 0), us + Slot::RSTD, Frag<float>{rs});
      bstore_frag<float>(rSV, keep_or_drop((16 * wave + n) * 16, lo == 0), us + Slot::CC, Frag<float>{cc});
      __syncthreads();  // G2 rows of every wave in
#pragma unroll
      for (int o = 0; o < FT; ++o) G2[o].v = sh.g2[o][l];
    } else {
      f4 tgt[FT];
#pragma unroll
      for (int q = 0; q < FT; ++q) {
        const Tile xkT = transpose16(xk[0][q], I);
        xkTf[q] = to_frag<T>(xkT.v);
        tgt[q] = transpose16(xv[q], I).v - xkT.v;
      }
      Tile z2[FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        z2[o].v = f4{b2_tm[o], b2_tm[o], b2_tm[o], b2_tm[o]};
#pragma unroll
        for (int w = 0; w < NW; ++w) z2[o].v += sh.z2p[w][o][l];
      }
      LnL2Lite<FT> ln;
      ln.forward(z2, tgt, lnw_tm, lnb_tm, eps, G2);
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        const int v = keep_or_drop(f4l + c * 1024, c % NW == wave);
        bstore_frag<float>(rSV, v, us + Slot::G2, Frag<float>{G2[c].v});
        bstore_frag<float>(rSV, v, us + Slot::XH, Frag<float>{ln.xh[c]});
      }
      bstore_frag<float>(rSV, keep_or_drop(f4l, wave == 0), us + Slot::RSTD, Frag<float>{ln.rstd});
      bstore_frag<float>(rSV, keep_or_drop(f4l, wave == 0), us + Slot::CC, Frag<float>{ln.c});
    }

    // ---- G1 = (G2 W2^T) (.) gelu'(Z1); W2^T blocks by exact transposes
    Tile G1[HT];
    {
      Frag<T> g2F[1][FT];  // feature-major frags of G2 (free = t, k = f)
#pragma unroll
      for (int o = 0; o < FT; ++o) g2F[0][o] = to_frag<T>(transpose16(to_frag<T>(G2[o].v), I).v);
#pragma unroll
      for (int i = 0; i < HT; ++i) {
        G1[i].v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q + 1 < FT; q += 2) {
          const Frag<T> t0 = to_frag<T>(transpose16(to_frag<T>(W2[i][q].v), I).v);
          const Frag<T> t1 = to_frag<T>(transpose16(to_frag<T>(W2[i][q + 1].v), I).v);
          mma32(G1[i].v, g2F[0][q], g2F[0][q + 1], t0, t1);
        }
        bstore_frag<T>(rSV, g1l + i * 256 * ST, us + Slot::H1, to_frag<T>(G1[i].v * gpp[i]));
        G1[i].v *= gp[i];
        bstore_frag<T>(rSV, g1l + i * 256 * ST, us + Slot::G1, to_frag<T>(G1[i].v));
      }
    }

    // ---- readout layer 1: Z1b = XQ W1 - (eta o A1 + eta) G1 + b1, X2b = gelu(Z1b)
    const f4 etaT = LR ? eta_rowfrag_from_lr(eta_rule, lr4) : frag_to_f4(etaTf);
    Frag<T> x2bF[1][HT];
    {
      Tile at[1][1];
      at[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      gemm<1, 1, FT>(at, xk, xq);  // (XQ XK^T)^T
      f4 m1;
#pragma unroll
      for (int j = 0; j < 4; ++j) m1[j] = -(etaT[j] * at[0][0].v[j] + etaT[j]);
      const Frag<T> m1f = to_frag<T>(m1);
      Tile zb[1][HT];
#pragma unroll
      for (int o = 0; o < HT; ++o) zb[0][o].v = f4{b1_tm[o], b1_tm[o], b1_tm[o], b1_tm[o]};
      gemm_pt<1, HT, FT>(zb, xq, W1);
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        mma16(zb[0][o].v, m1f, to_frag<T>(G1[o].v));
        f4 x2b, sp;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float y, dy;
          gelu_fwd_bwd(zb[0][o].v[j], y, dy);
          x2b[j] = y;
          sp[j] = dy;
        }
        bstore_frag<T>(rSV, g1l + o * 256 * ST, us + Slot::X2B, to_frag<T>(x2b));
        bstore_frag<T>(rSV, g1l + o * 256 * ST, us + Slot::SP1B, to_frag<T>(sp));
        x2bF[0][o] = to_frag<T>(transpose16(to_frag<T>(x2b), I).v);
      }
    }
    {
      Tile z2bp[1][FT], a2p[1][1];
#pragma unroll
      for (int o = 0; o < FT; ++o) z2bp[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
      a2p[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      gemm_pt<1, FT, HT>(z2bp, x2bF, W2);   // uses W2 before the update
      gemm<1, 1, HT>(a2p, x2F, x2bF);       // (X2b X2^T)^T over this wave's units
      if constexpr (kLnRowSplit<FT, NW>) {
        // Z2b = sum_w (X2b_w W2_w - (eta o A2_w) G2) - eta G2 + b2: the term
        // in A2 = sum_w A2_w is linear in it, so each wave adds its share and
        // wave 0 the rest; the sum of the partials is then Z2b itself
        f4 m2;
#pragma unroll
        for (int j = 0; j < 4; ++j) m2[j] = -(etaT[j] * a2p[0][0].v[j] + (wave == 0 ? etaT[j] : 0.f));
        const Frag<T> m2f = to_frag<T>(m2);
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          if (wave == 0) z2bp[0][o].v += f4{b2_tm[o], b2_tm[o], b2_tm[o], b2_tm[o]};
          mma16(z2bp[0][o].v, m2f, to_frag<T>(G2[o].v));
        }
      }
#pragma unroll
      for (int o = 0; o < FT; ++o) sh.z2bp[wave][o][l] = z2bp[0][o].v;
      sh.a2p[wave][l] = a2p[0][0].v;
    }
    const f4 e = LR ? eta_lastrow_from_lr(lr4) : frag_to_f4(ef);

    // ---- state update (the readout above used the state entering s)
    float b2_old[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) b2_old[o] = b2_tm[o];
    {
      Frag<T> g1e[HT], g2e[FT];
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        f4 v;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = -e[j] * G1[o].v[j];
          acc += e[j] * G1[o].v[j];
        }
        g1e[o] = to_frag<T>(v);
        const float d = sum_col4(acc);
        b1_tm[o] -= d;
        bstore_frag<T>(rSV, g1l + o * 256 * ST, us + Slot::G1E, g1e[o]);
        bstore_f32(rSV, (hs + n) * 4 + 64 * o, us + Slot::B1D, d);  // the 4 lanes of column n agree
      }
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        f4 v;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = -e[j] * G2[o].v[j];
          acc += e[j] * G2[o].v[j];
        }
        g2e[o] = to_frag<T>(v);
        const float d = sum_col4(acc);
        b2_tm[o] -= d;
        bstore_frag<T>(rSV, keep_or_drop(g2l + o * 256 * ST, wave == 0), us + Slot::G2E, g2e[o]);
        bstore_f32(rSV, keep_or_drop(n * 4 + 64 * o, wave == 0), us + Slot::B2D, d);
      }
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < HT; ++o) mma16(W1[i][o].v, xkTf[i], g1e[o]);
#pragma unroll
      for (int i = 0; i < HT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) mma16(W2[i][o].v, x2f[i], g2e[o]);
    }
    __syncthreads();

    // ---- readout layer 2, LayerNorm, residual
    if constexpr (kLnRowSplit<FT, NW>) {
      // rows 4*wave + j, feature l, as in the inner loss's LayerNorm; the
      // last wave, which has no bias share above, saves A2
      if (wave == NW - 1) {
        f4 a2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; ++w) a2 += sh.a2p[w][l];
        bstore_tile(rSV, a2l, us + Slot::A2T, 16, 0, 0, Tile{a2});
      }
      const int lo = l >> 4;
      f4 z = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NW; ++w) z += sh.z2bp[w][lo][16 * wave + n];
      constexpr float invF = 1.0f / F;
      const f4 mu = sum4_wave(z) * invF;
      const f4 d = z - mu;
      const f4 var = sum4_wave(d * d) * invF;
      const f4 q = frag_to_f4(xqr);
      f4 rs, xhb, y;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        rs[j] = rsqrt_f(var[j] + eps);
        xhb[j] = d[j] * rs[j];
        y[j] = q[j] + lnw_l * xhb[j] + lnb_l;
      }
      bstore_frag<float>(rSV, keep_or_drop((16 * wave + n) * 16, lo == 0), us + Slot::RSB, Frag<float>{rs});
      bstore_frag<float>(rSV, (lo * 64 + 16 * wave + n) * 16, us + Slot::XHB, Frag<float>{xhb});
      bstore_ctile<T>(rOUT, l * ST, xo + 4 * wave * F * ST, F, to_frag<T>(y));
    } else {
      Tile a2[1];
      a2[0].v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NW; ++w) a2[0].v += sh.a2p[w][l];
      bstore_tile(rSV, keep_or_drop(a2l, wave == 0), us + Slot::A2T, 16, 0, 0, a2[0]);
      f4 m2;
#pragma unroll
      for (int j = 0; j < 4; ++j) m2[j] = -(etaT[j] * a2[0].v[j] + etaT[j]);
      const Frag<T> m2f = to_frag<T>(m2);
      Tile z2b[FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        z2b[o].v = f4{b2_old[o], b2_old[o], b2_old[o], b2_old[o]};
#pragma unroll
        for (int w = 0; w < NW; ++w) z2b[o].v += sh.z2bp[w][o][l];
        mma16(z2b[o].v, m2f, to_frag<T>(G2[o].v));
      }
      // LayerNorm over features of each token row (token-major)
      constexpr float invF = 1.0f / F;
      f4 mu, rs;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int o = 0; o < FT; ++o) acc += z2b[o].v[j];
        mu[j] = sum_row16(acc) * invF;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          const float d = z2b[o].v[j] - mu[j];
          acc += d * d;
        }
        rs[j] = rsqrt_f(sum_row16(acc) * invF + eps);
      }
      bstore_frag<float>(rSV, keep_or_drop(f4l, wave == 0), us + Slot::RSB, Frag<float>{rs});
      if constexpr (NW == FT) {
        // one tile per wave: tile o = wave, picked out of the register arrays
        // by uniform selects
        const int o = wave;
        f4 zo = z2b[0].v;
        Frag<T> xqo = xq[0][0];
#pragma unroll
        for (int c = 1; c < FT; ++c) {
          if (o == c) {
            zo = z2b[c].v;
            xqo = xq[0][c];
          }
        }
        const f4 q = transpose16(xqo, I).v;  // XQ token-major
        f4 xhb, y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xhb[j] = (zo[j] - mu[j]) * rs[j];
          y[j] = q[j] + lnw_own * xhb[j] + lnb_own;
        }
        bstore_frag<float>(rSV, f4l + o * 1024, us + Slot::XHB, Frag<float>{xhb});
        bstore_frag<T>(rOUT, xl + 16 * o * ST, xo, to_frag<T>(transpose16(to_frag<T>(y), I).v));
      } else {
        // every wave forms every tile; tile o is written by wave o % NW
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          const bool mine = o % NW == wave;
          const f4 q = transpose16(xq[0][o], I).v;  // XQ token-major
          f4 xhb, y;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            xhb[j] = (z2b[o].v[j] - mu[j]) * rs[j];
            y[j] = q[j] + lnw_tm[o] * xhb[j] + lnb_tm[o];
          }
          bstore_frag<float>(rSV, keep_or_drop(f4l + o * 1024, mine), us + Slot::XHB, Frag<float>{xhb});
          bstore_frag<T>(rOUT, keep_or_drop(xl + 16 * o * ST, mine), xo,
                         to_frag<T>(transpose16(to_frag<T>(y), I).v));
        }
      }
    }

    if (p.W1_memo != nullptr && (s % p.M) == 0) {
      const size_t k = (size_t)chain * p.NS + s / p.M;
      store_state(p.W1_memo + k * F * FF, p.b1_memo + k * FF, p.W2_memo + k * FF * F, p.b2_memo + k * F);
    }
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      xq[0][q] = xqn[q];
      xk[0][q] = xkn[q];
    }
  }

  if (p.W1_last != nullptr) {
    store_state(p.W1_last + (size_t)chain * F * FF, p.b1_last + (size_t)chain * FF, p.W2_last + (size_t)chain * FF * F,
                p.b2_last + (size_t)chain * F);
  }
}

template <typename T, int FT, int NW, int HT>
static hipError_t launch_mlp_fwd_t(const MlpFwdParams& p, hipStream_t stream) {
  static_assert(MlpSavedSlot<16 * FT, 16 * HT * NW, (int)sizeof(T)>::BYTES ==
                    (int)mlp_saved_slot_bytes_of(16 * FT, 16 * HT * NW, (int)sizeof(T)),
                "saved slot layout");
  if (p.eta_rule == TTT_ETA_DENSE)
    hipLaunchKernelGGL((mlp_fwd_kernel<T, FT, NW, HT, false>), dim3(p.B * p.H), dim3(64 * NW), 0, stream, p);
  else if (p.eta_rule == TTT_ETA_DENSE_F32)
    hipLaunchKernelGGL((mlp_fwd_kernel<T, FT, NW, HT, false, float>), dim3(p.B * p.H), dim3(64 * NW), 0, stream, p);
  else
    hipLaunchKernelGGL((mlp_fwd_kernel<T, FT, NW, HT, true>), dim3(p.B * p.H), dim3(64 * NW), 0, stream, p);
  return hipGetLastError();
}

template <typename T, int FT>
static hipError_t launch_mlp_fwd_f(const MlpFwdParams& p, hipStream_t stream) {
  switch (p.FF) {
    case 64:  // at F = 64 four waves of FF/64 hidden tiles, so that the LayerNorms split by rows
      if constexpr (FT == 4) return launch_mlp_fwd_t<T, FT, 4, 1>(p, stream);
      else return launch_mlp_fwd_t<T, FT, 1, 4>(p, stream);
    case 128:
      if constexpr (FT == 4) return launch_mlp_fwd_t<T, FT, 4, 2>(p, stream);
      else return launch_mlp_fwd_t<T, FT, 2, 4>(p, stream);
    case 256: return launch_mlp_fwd_t<T, FT, 4, 4>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_mlp_fwd(const MlpFwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_mlp_fwd_f<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_mlp_fwd_f<__bf16, 2>(p, stream);
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_mlp_fwd_f<_Float16, 4>(p, stream);
    if (p.F == 32) return launch_mlp_fwd_f<_Float16, 2>(p, stream);
  } else {
    if (p.F == 64) return launch_mlp_fwd_f<float, 4>(p, stream);
    if (p.F == 32) return launch_mlp_fwd_f<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
