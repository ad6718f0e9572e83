// TTT-MLP backward on gfx950: one workgroup of NW = FF/64 wavefronts per
// (batch, head) chain; wave w owns hidden units S = [64w, 64w+64).
//
// Reverse sweep over checkpoint groups (kernels/mlp_backward.py:340 walks the
// same groups; the algorithm and data flow here are our own):
//   pass 1  reload the state entering the group from its checkpoint and run
//           the group's mini-batches forward (state path only).  Before each
//           mini-batch the state's MFMA operand values (W1 and W2 in both
//           orientations, in the activation dtype, plus b1, b2 in fp32) are
//           written to the per-chain workspace, so pass 2 can load any operand
//           frag with contiguous 4-element reads.  While pass 1 holds the
//           state in registers, the gradient accumulators dW1, dW2 are parked
//           in LDS.
//   pass 2  walk the group backwards: recompute the mini-batch forward from
//           the stored operands and apply its gradient (ops/ttt_mlp.py:9-67
//           differentiated by hand), with dW1 = dL/dW1', dW2, db1, db2 (the
//           gradient wrt the state after the mini-batch) in registers.
// Row-wise work on [16 x F] tiles (LayerNorms and their backward) is done
// redundantly by every wave; contractions over the hidden units are split by
// slice and reduced through LDS (five barriers per mini-batch).
#include "ttt_kernels.h"
#include "ttt_ln.h"

namespace ttt {

template <typename T, int FT, int NW> struct MlpBwdShared {
  static constexpr int HT = 4;
  f4 partZ[NW][FT][64];                       // Z2 partials (both passes)
  union {
    f4 park[NW][2 * FT * HT][64];             // pass 1: parked dW1, dW2 tiles
    struct {
      f4 partA[NW][FT][64];                   // dXQ partials
      f4 partB[NW][FT][64];                   // Z2b partials, then dG2 partials
      f4 partC[NW][FT][64];                   // Q2 partials, then dXK partials
      f4 partD[NW][FT][64];                   // -(e G1) dW1'^T partials
      f4 a2T[NW][64], a2[NW][64];             // (X2b X2^T) partials, both layouts
      f4 dn1[NW][64], dn1T[NW][64];           // dN1 partials, both layouts
      f4 de[NW][64];                          // eta-row gradient partials
    } s;
  } u;
};

template <typename T> __device__ __forceinline__ void store4(T* __restrict__ p, f4 v);
template <> __device__ __forceinline__ void store4<__bf16>(__bf16* __restrict__ p, f4 v) {
  *reinterpret_cast<bf4*>(p) = to_frag<__bf16>(v).v;
}
template <> __device__ __forceinline__ void store4<float>(float* __restrict__ p, f4 v) {
  *reinterpret_cast<f4*>(p) = v;
}

template <typename T, int FT, int NW>
__global__ __launch_bounds__(64 * NW) void mlp_bwd_kernel(MlpBwdParams p) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  constexpr int HT = 4;
  constexpr int FF = 64 * NW;
  constexpr float invF = 1.0f / F;
  __shared__ MlpBwdShared<T, FT, NW> sh;

  const int chain = blockIdx.x;
  const int h = chain % p.H;
  const int NC = p.NC, G = p.G, NK = p.NK;
  const int wave = threadIdx.x >> 6;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  const int hs = 64 * wave;

  const size_t xoff = (size_t)chain * NC * K * F;
  const size_t eoff = (size_t)chain * NC * K * K;
  const T* __restrict__ XQ = static_cast<const T*>(p.XQ) + xoff;
  const T* __restrict__ XK = static_cast<const T*>(p.XK) + xoff;
  const T* __restrict__ XV = static_cast<const T*>(p.XV) + xoff;
  const T* __restrict__ DO = static_cast<const T*>(p.dout) + xoff;
  const T* __restrict__ ETA = static_cast<const T*>(p.eta) + eoff;
  T* __restrict__ DXQ = static_cast<T*>(p.dXQ) + xoff;
  T* __restrict__ DXK = static_cast<T*>(p.dXK) + xoff;
  T* __restrict__ DXV = static_cast<T*>(p.dXV) + xoff;
  T* __restrict__ DETA = static_cast<T*>(p.deta) + eoff;
  // workspace slot: W1t [FF][F], W2t [F][FF], W1 [F][FF], W2 [FF][F] (T), b1 [FF], b2 [F] (fp32)
  const size_t mat = (size_t)F * FF;
  const size_t slot_bytes = 4 * mat * sizeof(T) + (FF + F) * sizeof(float);
  char* WSB = reinterpret_cast<char*>(p.ws) + (size_t)chain * G * slot_bytes;

  float lnw_tm[FT], lnb_tm[FT];
#pragma unroll
  for (int o = 0; o < FT; ++o) {
    lnw_tm[o] = p.ln_w[h * F + 16 * o + n];
    lnb_tm[o] = p.ln_b[h * F + 16 * o + n];
  }
  const float eps = p.eps;
  const Frag<T> I = identity_frag<T>();

  // gradient wrt the state after the current mini-batch (this wave's slice)
  Tile dW1[FT][HT], dW2[HT][FT];
  float db1[HT], db2[FT];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < HT; ++o) {
      dW1[i][o].v = f4{0.f, 0.f, 0.f, 0.f};
      dW2[o][i].v = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
  for (int o = 0; o < HT; ++o) db1[o] = 0.f;
#pragma unroll
  for (int o = 0; o < FT; ++o) db2[o] = 0.f;
  float dlnw[FT], dlnb[FT];  // LN-parameter gradient partials (wave 0)
#pragma unroll
  for (int o = 0; o < FT; ++o) {
    dlnw[o] = 0.f;
    dlnb[o] = 0.f;
  }

  for (int kk = NK - 1; kk >= 0; --kk) {
    const int s0 = kk * G, s1 = min(s0 + G, NC);

    // ===================== pass 1: advance the state, store operands
    __syncthreads();  // LDS partials of the previous group are consumed
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        sh.u.park[wave][i * HT + o][l] = dW1[i][o].v;
        sh.u.park[wave][FT * HT + o * FT + i][l] = dW2[o][i].v;
      }
    {
      Tile W1[FT][HT], W2[HT][FT];
      float b1[HT], b2[FT];
      {
        const size_t k = (size_t)chain * NK + kk;
        const float* w1 = p.W1_ckpt + k * F * FF;
        const float* w2 = p.W2_ckpt + k * FF * F;
#pragma unroll
        for (int i = 0; i < FT; ++i)
#pragma unroll
          for (int o = 0; o < HT; ++o) W1[i][o] = load_tile(w1, FF, 16 * i, hs + 16 * o);
#pragma unroll
        for (int i = 0; i < HT; ++i)
#pragma unroll
          for (int o = 0; o < FT; ++o) W2[i][o] = load_tile(w2, F, hs + 16 * i, 16 * o);
#pragma unroll
        for (int o = 0; o < HT; ++o) b1[o] = p.b1_ckpt[k * FF + hs + 16 * o + n];
#pragma unroll
        for (int o = 0; o < FT; ++o) b2[o] = p.b2_ckpt[k * F + 16 * o + n];
      }
      for (int s = s0; s < s1; ++s) {
        char* slot = WSB + (size_t)(s - s0) * slot_bytes;
        T* W1t_ = reinterpret_cast<T*>(slot);
        T* W2t_ = W1t_ + mat;
        T* W1_ = W2t_ + mat;
        T* W2_ = W1_ + mat;
        float* b1_ = reinterpret_cast<float*>(W2_ + mat);
        float* b2_ = b1_ + FF;
#pragma unroll
        for (int i = 0; i < FT; ++i)
#pragma unroll
          for (int o = 0; o < HT; ++o) {
            // W1 tile rows f = 16i+4g+j, cols hs+16o+n
            store4<T>(W1t_ + (size_t)(hs + 16 * o + n) * F + 16 * i + 4 * g, W1[i][o].v);
            store4<T>(W1_ + (size_t)(16 * i + n) * FF + hs + 16 * o + 4 * g,
                      transpose16(to_frag<T>(W1[i][o].v), I).v);
          }
#pragma unroll
        for (int i = 0; i < HT; ++i)
#pragma unroll
          for (int o = 0; o < FT; ++o) {
            // W2 tile rows hs+16i+4g+j, cols f = 16o+n
            store4<T>(W2t_ + (size_t)(16 * o + n) * FF + hs + 16 * i + 4 * g, W2[i][o].v);
            store4<T>(W2_ + (size_t)(hs + 16 * i + n) * F + 16 * o + 4 * g,
                      transpose16(to_frag<T>(W2[i][o].v), I).v);
          }
        if (g == 0) {
#pragma unroll
          for (int o = 0; o < HT; ++o) b1_[hs + 16 * o + n] = b1[o];
          if (wave == 0) {
#pragma unroll
            for (int o = 0; o < FT; ++o) b2_[16 * o + n] = b2[o];
          }
        }
        if (s == s1 - 1) break;  // the state after the group is not needed

        // state path of the forward (mlp_fwd_kernel without the readout)
        const size_t xo = (size_t)s * K * F;
        Frag<T> xk[1][FT], xkTf[FT];
        f4 tgt[FT];
#pragma unroll
        for (int q = 0; q < FT; ++q) {
          xk[0][q] = load_frag(XK + xo, F, 16 * q);
          const Tile xkT = transpose16(xk[0][q], I);
          xkTf[q] = to_frag<T>(xkT.v);
          tgt[q] = transpose16(load_frag(XV + xo, F, 16 * q), I).v - xkT.v;
        }
        Frag<T> x2f[HT], x2F[1][HT];
        f4 gp[HT];
        {
          Tile z1[1][HT];
#pragma unroll
          for (int o = 0; o < HT; ++o) z1[0][o].v = f4{b1[o], b1[o], b1[o], b1[o]};
          gemm_pt<1, HT, FT>(z1, xk, W1);
#pragma unroll
          for (int o = 0; o < HT; ++o) {
            f4 x2;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              x2[j] = gelu_tanh(z1[0][o].v[j]);
              gp[o][j] = gelu_bwd(z1[0][o].v[j]);
            }
            x2f[o] = to_frag<T>(x2);
            x2F[0][o] = to_frag<T>(transpose16(x2f[o], I).v);
          }
        }
        {
          Tile z2p[1][FT];
#pragma unroll
          for (int o = 0; o < FT; ++o) z2p[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
          gemm_pt<1, FT, HT>(z2p, x2F, W2);
#pragma unroll
          for (int o = 0; o < FT; ++o) sh.partZ[wave][o][l] = z2p[0][o].v;
        }
        __syncthreads();
        Tile G2[FT];
        {
          Tile z2[FT];
#pragma unroll
          for (int o = 0; o < FT; ++o) {
            z2[o].v = f4{b2[o], b2[o], b2[o], b2[o]};
#pragma unroll
            for (int w = 0; w < NW; ++w) z2[o].v += sh.partZ[w][o][l];
          }
          LnL2TM<FT> ln;
          ln.forward(z2, tgt, lnw_tm, lnb_tm, eps, G2);
        }
        __syncthreads();  // partZ is rewritten by the next mini-batch
        Tile G1[HT];
        {
          Frag<T> g2F[1][FT];
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
            G1[i].v *= gp[i];
          }
        }
        const f4 e = load4(ETA + (size_t)s * K * K + (K - 1) * K + 4 * g);
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
          b1[o] -= sum_col4(acc);
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
          b2[o] -= sum_col4(acc);
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
    }
    __syncthreads();  // workspace written; parked dW visible
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        dW1[i][o].v = sh.u.park[wave][i * HT + o][l];
        dW2[o][i].v = sh.u.park[wave][FT * HT + o * FT + i][l];
      }
    __syncthreads();  // park area is reused for pass-2 partials

    // ===================== pass 2: reverse through the group
    for (int s = s1 - 1; s >= s0; --s) {
      const char* slot = WSB + (size_t)(s - s0) * slot_bytes;
      const T* W1t_ = reinterpret_cast<const T*>(slot);
      const T* W2t_ = W1t_ + mat;
      const T* W1_ = W2t_ + mat;
      const T* W2_ = W1_ + mat;
      const float* b1_ = reinterpret_cast<const float*>(W2_ + mat);
      const float* b2_ = b1_ + FF;
      const size_t xo = (size_t)s * K * F;
      const T* etas = ETA + (size_t)s * K * K;

      Frag<T> xq[1][FT], xk[1][FT];
#pragma unroll
      for (int q = 0; q < FT; ++q) {
        xq[0][q] = load_frag(XQ + xo, F, 16 * q);
        xk[0][q] = load_frag(XK + xo, F, 16 * q);
      }
      float b1s[HT], b2s[FT];
#pragma unroll
      for (int o = 0; o < HT; ++o) b1s[o] = b1_[hs + 16 * o + n];
#pragma unroll
      for (int o = 0; o < FT; ++o) b2s[o] = b2_[16 * o + n];

      // ---- R1: layer 1 (Z1 for this slice) and XQ W1
      Frag<T> x2f[HT], x2F[1][HT];
      f4 sp1[HT], spp1[HT];
      Tile zq[1][HT];
      {
        Frag<T> w1t[HT][FT];  // (free = hidden, k = f)
#pragma unroll
        for (int o = 0; o < HT; ++o)
#pragma unroll
          for (int q = 0; q < FT; ++q) w1t[o][q] = load_frag(W1t_ + (size_t)(hs + 16 * o) * F, F, 16 * q);
        Tile z1[1][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          z1[0][o].v = f4{b1s[o], b1s[o], b1s[o], b1s[o]};
          zq[0][o].v = f4{b1s[o], b1s[o], b1s[o], b1s[o]};
        }
        gemm<1, HT, FT>(z1, xk, w1t);
        gemm<1, HT, FT>(zq, xq, w1t);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          f4 x2;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float z = z1[0][o].v[j];
            x2[j] = gelu_tanh(z);
            sp1[o][j] = gelu_bwd(z);
            spp1[o][j] = gelu_bwd2(z);
          }
          x2f[o] = to_frag<T>(x2);
          x2F[0][o] = to_frag<T>(transpose16(x2f[o], I).v);
        }
      }
      // ---- R2: Z2 partial over this slice
      {
        Frag<T> w2t[FT][HT];  // (free = f, k = hidden)
#pragma unroll
        for (int o = 0; o < FT; ++o)
#pragma unroll
          for (int c = 0; c < HT; ++c) w2t[o][c] = load_frag(W2t_ + (size_t)(16 * o) * FF, FF, hs + 16 * c);
        Tile z2p[1][FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) z2p[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, FT, HT>(z2p, x2F, w2t);
#pragma unroll
        for (int o = 0; o < FT; ++o) sh.partZ[wave][o][l] = z2p[0][o].v;
      }
      __syncthreads();  // (1)

      // ---- R3: G2 (every wave), G1 and the readout of layer 1 (per slice)
      Frag<T> xkTf[FT], xqTf[FT];
      LnL2TM<FT> ln2;
      Tile G2[FT];
      {
        f4 tgt[FT];
#pragma unroll
        for (int q = 0; q < FT; ++q) {
          const Tile xkT = transpose16(xk[0][q], I);
          xkTf[q] = to_frag<T>(xkT.v);
          xqTf[q] = to_frag<T>(transpose16(xq[0][q], I).v);
          tgt[q] = transpose16(load_frag(XV + xo, F, 16 * q), I).v - xkT.v;
        }
        Tile z2[FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          z2[o].v = f4{b2s[o], b2s[o], b2s[o], b2s[o]};
#pragma unroll
          for (int w = 0; w < NW; ++w) z2[o].v += sh.partZ[w][o][l];
        }
        ln2.forward(z2, tgt, lnw_tm, lnb_tm, eps, G2);
      }
      Frag<T> g2F[1][FT], g2f[FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        g2f[o] = to_frag<T>(G2[o].v);
        g2F[0][o] = to_frag<T>(transpose16(g2f[o], I).v);
      }
      Frag<T> w2[HT][FT];  // (free = hidden, k = f)
#pragma unroll
      for (int i = 0; i < HT; ++i)
#pragma unroll
        for (int q = 0; q < FT; ++q) w2[i][q] = load_frag(W2_ + (size_t)(hs + 16 * i) * F, F, 16 * q);
      Tile Pm[1][HT];
#pragma unroll
      for (int i = 0; i < HT; ++i) Pm[0][i].v = f4{0.f, 0.f, 0.f, 0.f};
      gemm<1, HT, FT>(Pm, g2F, w2);
      Tile G1[HT];
#pragma unroll
      for (int i = 0; i < HT; ++i) G1[i].v = Pm[0][i].v * sp1[i];

      const f4 etaT = load_f4(etas, K, 0);  // [t_k x t_q]: eta[n][4g+j]
      f4 eta_n;                             // [t_q x t_k]: eta[4g+j][n]
#pragma unroll
      for (int j = 0; j < 4; ++j) eta_n[j] = (float)etas[(4 * g + j) * K + n];
      const f4 e = load4(etas + (K - 1) * K + 4 * g);
      Tile at[1][1], a[1][1];
      at[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      a[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      gemm<1, 1, FT>(at, xk, xq);  // A1^T [t_k x t_q]
      gemm<1, 1, FT>(a, xq, xk);   // A1   [t_q x t_k]
      f4 m1T, m1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m1T[j] = etaT[j] * at[0][0].v[j] + etaT[j];
        m1[j] = eta_n[j] * a[0][0].v[j] + eta_n[j];
      }
      Frag<T> x2bf[HT], x2bF[1][HT];
      f4 sp1b[HT];
      {
        const Frag<T> mnf = to_frag<T>(-m1T);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          mma16(zq[0][o].v, mnf, to_frag<T>(G1[o].v));  // Z1b = XQ W1 + b1 - M1 G1
          f4 x2b;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            x2b[j] = gelu_tanh(zq[0][o].v[j]);
            sp1b[o][j] = gelu_bwd(zq[0][o].v[j]);
          }
          x2bf[o] = to_frag<T>(x2b);
          x2bF[0][o] = to_frag<T>(transpose16(x2bf[o], I).v);
        }
      }
      {
        Frag<T> w2t[FT][HT];
#pragma unroll
        for (int o = 0; o < FT; ++o)
#pragma unroll
          for (int c = 0; c < HT; ++c) w2t[o][c] = load_frag(W2t_ + (size_t)(16 * o) * FF, FF, hs + 16 * c);
        Tile z2bp[1][FT], a2Tp[1][1], a2p[1][1];
#pragma unroll
        for (int o = 0; o < FT; ++o) z2bp[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
        a2Tp[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
        a2p[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, FT, HT>(z2bp, x2bF, w2t);
        gemm<1, 1, HT>(a2Tp, x2F, x2bF);  // A2^T [t_k x t_q]
        gemm<1, 1, HT>(a2p, x2bF, x2F);   // A2   [t_q x t_k]
#pragma unroll
        for (int o = 0; o < FT; ++o) sh.u.s.partB[wave][o][l] = z2bp[0][o].v;
        sh.u.s.a2T[wave][l] = a2Tp[0][0].v;
        sh.u.s.a2[wave][l] = a2p[0][0].v;
      }
      __syncthreads();  // (2)

      // ---- R4: readout layer 2 and its LayerNorm backward (every wave)
      f4 a2T = f4{0.f, 0.f, 0.f, 0.f}, a2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        a2T += sh.u.s.a2T[w][l];
        a2 += sh.u.s.a2[w][l];
      }
      f4 m2T, m2;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m2T[j] = etaT[j] * a2T[j] + etaT[j];
        m2[j] = eta_n[j] * a2[j] + eta_n[j];
      }
      Frag<T> dz2bf[FT], dz2bF[1][FT];
      float dz2b_cs[FT];  // column sums of dZ2b (fp32)
      {
        Tile z2b[FT];
        const Frag<T> mnf = to_frag<T>(-m2T);
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          z2b[o].v = f4{b2s[o], b2s[o], b2s[o], b2s[o]};
#pragma unroll
          for (int w = 0; w < NW; ++w) z2b[o].v += sh.u.s.partB[w][o][l];
          mma16(z2b[o].v, mnf, g2f[o]);
        }
        f4 mb, rsb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float acc = 0.f;
#pragma unroll
          for (int o = 0; o < FT; ++o) acc += z2b[o].v[j];
          mb[j] = sum_row16(acc) * invF;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float acc = 0.f;
#pragma unroll
          for (int o = 0; o < FT; ++o) {
            const float d = z2b[o].v[j] - mb[j];
            acc += d * d;
          }
          rsb[j] = 1.0f / sqrtf(sum_row16(acc) * invF + eps);
        }
        f4 dT[FT], xhb[FT], gy[FT];
        f4 a1 = f4{0.f, 0.f, 0.f, 0.f}, a2s = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          dT[o] = transpose16(load_frag(DO + xo, F, 16 * o), I).v;  // dout, token-major
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            xhb[o][j] = (z2b[o].v[j] - mb[j]) * rsb[j];
            gy[o][j] = dT[o][j] * lnw_tm[o];
            a1[j] += gy[o][j];
            a2s[j] += gy[o][j] * xhb[o][j];
          }
          if (wave == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              dlnw[o] += dT[o][j] * xhb[o][j];
              dlnb[o] += dT[o][j];
            }
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a1[j] = sum_row16(a1[j]) * invF;
          a2s[j] = sum_row16(a2s[j]) * invF;
        }
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          f4 dz;
          float cs = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dz[j] = rsb[j] * (gy[o][j] - a1[j] - xhb[o][j] * a2s[j]);
            cs += dz[j];
          }
          dz2b_cs[o] = sum_col4(cs);
          dz2bf[o] = to_frag<T>(dz);
          dz2bF[0][o] = to_frag<T>(transpose16(dz2bf[o], I).v);
        }
      }
      // dN2 = -dZ2b G2^T (both layouts), deta part, dA2; dG2 = -M2^T dZ2b
      f4 detT, dA2T, dA2;
      {
        Tile dn[1][1], dnT[1][1];
        dn[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
        dnT[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, 1, FT>(dn, dz2bF, g2F);   // dZ2b G2^T [t_q x t_k]
        gemm<1, 1, FT>(dnT, g2F, dz2bF);  // G2 dZ2b^T [t_k x t_q]
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          detT[j] = -dnT[0][0].v[j] * (1.0f + a2T[j]);
          dA2T[j] = -dnT[0][0].v[j] * etaT[j];
          dA2[j] = -dn[0][0].v[j] * eta_n[j];
        }
      }
      Tile dG2[FT];
      {
        const Frag<T> mf = to_frag<T>(-m2);
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          dG2[o].v = f4{0.f, 0.f, 0.f, 0.f};
          mma16(dG2[o].v, mf, dz2bf[o]);
        }
      }

      // ---- B1: readout layer 1 backward and the state-update terms (per slice)
      Frag<T> dz1bf[HT], dz1bF[1][HT];
      float dz1b_cs[HT];  // column sums of dZ1b (fp32)
      Tile dX2[HT], dG1[HT];
      {
        Tile dx2b[1][HT];
#pragma unroll
        for (int i = 0; i < HT; ++i) dx2b[0][i].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, HT, FT>(dx2b, dz2bF, w2);  // dZ2b W2^T
        const Frag<T> dA2Tf = to_frag<T>(dA2T), dA2f = to_frag<T>(dA2);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          mma16(dx2b[0][o].v, dA2Tf, x2f[o]);  // + dA2 X2
          const f4 dz = dx2b[0][o].v * sp1b[o];
          dz1b_cs[o] = sum_col4(dz[0] + dz[1] + dz[2] + dz[3]);
          dz1bf[o] = to_frag<T>(dz);
          dz1bF[0][o] = to_frag<T>(transpose16(dz1bf[o], I).v);
          dX2[o].v = f4{0.f, 0.f, 0.f, 0.f};
          mma16(dX2[o].v, dA2f, x2bf[o]);      // dA2^T X2b
        }
      }
      {
        Frag<T> g1F[1][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) g1F[0][o] = to_frag<T>(transpose16(to_frag<T>(G1[o].v), I).v);
        Tile dn[1][1], dnT[1][1];
        dn[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
        dnT[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, 1, HT>(dn, dz1bF, g1F);
        gemm<1, 1, HT>(dnT, g1F, dz1bF);
        sh.u.s.dn1[wave][l] = dn[0][0].v;
        sh.u.s.dn1T[wave][l] = dnT[0][0].v;
        // -(e G1) dW1'^T over this slice -> dXK partial
        Frag<T> eg1F[1][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          f4 v;
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = -e[j] * G1[o].v[j];
          eg1F[0][o] = to_frag<T>(transpose16(to_frag<T>(v), I).v);
        }
        Tile t1[1][FT];
#pragma unroll
        for (int q = 0; q < FT; ++q) {
          t1[0][q].v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < HT; c += 2) {
            const Frag<T> u0 = to_frag<T>(transpose16(to_frag<T>(dW1[q][c].v), I).v);
            const Frag<T> u1 = to_frag<T>(transpose16(to_frag<T>(dW1[q][c + 1].v), I).v);
            mma32(t1[0][q].v, eg1F[0][c], eg1F[0][c + 1], u0, u1);
          }
          sh.u.s.partD[wave][q][l] = t1[0][q].v;
        }
      }
      {
        Frag<T> w1[FT][HT];  // (free = f, k = hidden)
#pragma unroll
        for (int o = 0; o < FT; ++o)
#pragma unroll
          for (int c = 0; c < HT; ++c) w1[o][c] = load_frag(W1_ + (size_t)(16 * o) * FF, FF, hs + 16 * c);
        Tile dxqp[1][FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) dxqp[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, FT, HT>(dxqp, dz1bF, w1);  // dZ1b W1^T
#pragma unroll
        for (int o = 0; o < FT; ++o) sh.u.s.partA[wave][o][l] = dxqp[0][o].v;
      }
      {
        // dG1 = -M1^T dZ1b - e (XK dW1' + db1')
        Tile q1[1][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) q1[0][o].v = f4{db1[o], db1[o], db1[o], db1[o]};
        gemm_pt<1, HT, FT>(q1, xk, dW1);
        const Frag<T> mf = to_frag<T>(-m1);
        f4 dep = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          dG1[o].v = f4{0.f, 0.f, 0.f, 0.f};
          mma16(dG1[o].v, mf, dz1bf[o]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dG1[o].v[j] -= e[j] * q1[0][o].v[j];
            dep[j] += G1[o].v[j] * q1[0][o].v[j];
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) dep[j] = sum_row16(dep[j]);
        sh.u.s.de[wave][l] = dep;
        // X2 dW2' over this slice -> Q2 partial
        Tile q2p[1][FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) q2p[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm_pt<1, FT, HT>(q2p, x2F, dW2);
#pragma unroll
        for (int o = 0; o < FT; ++o) sh.u.s.partC[wave][o][l] = q2p[0][o].v;
        // dX2 -= (e G2) dW2'^T  (contraction over f, dW2'^T frags by transposes)
        Frag<T> eg2F[1][FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          f4 v;
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = -e[j] * G2[o].v[j];
          eg2F[0][o] = to_frag<T>(transpose16(to_frag<T>(v), I).v);
        }
#pragma unroll
        for (int c = 0; c < HT; ++c)
#pragma unroll
          for (int q = 0; q + 1 < FT; q += 2) {
            const Frag<T> u0 = to_frag<T>(transpose16(to_frag<T>(dW2[c][q].v), I).v);
            const Frag<T> u1 = to_frag<T>(transpose16(to_frag<T>(dW2[c][q + 1].v), I).v);
            mma32(dX2[c].v, eg2F[0][q], eg2F[0][q + 1], u0, u1);
          }
      }
      __syncthreads();  // (3)

      // ---- B2: assemble dN1, Q2, de; dXQ and deta (wave 0); dP, dZ1
      f4 dn1 = f4{0.f, 0.f, 0.f, 0.f}, dn1T = f4{0.f, 0.f, 0.f, 0.f}, de = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        dn1 += sh.u.s.dn1[w][l];
        dn1T += sh.u.s.dn1T[w][l];
        de += sh.u.s.de[w][l];
      }
      f4 dA1T, dA1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dn1[j] = -dn1[j];
        dn1T[j] = -dn1T[j];
        detT[j] += dn1T[j] * (1.0f + at[0][0].v[j]);
        dA1T[j] = dn1T[j] * etaT[j];
        dA1[j] = dn1[j] * eta_n[j];
      }
      {
        f4 dep = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          f4 q2 = f4{db2[o], db2[o], db2[o], db2[o]};
#pragma unroll
          for (int w = 0; w < NW; ++w) q2 += sh.u.s.partC[w][o][l];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dG2[o].v[j] -= e[j] * q2[j];
            dep[j] += G2[o].v[j] * q2[j];
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) de[j] = -(de[j] + sum_row16(dep[j]));
      }
      if (wave == 0) {
        const Frag<T> dA1Tf = to_frag<T>(dA1T);
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          Tile dxq;
          dxq.v = transpose16(load_frag(DO + xo, F, 16 * o), I).v;
#pragma unroll
          for (int w = 0; w < NW; ++w) dxq.v += sh.u.s.partA[w][o][l];
          mma16(dxq.v, dA1Tf, xkTf[o]);  // + dA1 XK
          store_f4(DXQ + xo, F, 16 * o, transpose16(to_frag<T>(dxq.v), I).v);
        }
        if (n == K - 1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) detT[j] += de[j];
        }
        store_f4(DETA + (size_t)s * K * K, K, 0, detT);
      }
      Frag<T> dPf[HT];
      Tile dZ1[HT];
      {
        Frag<T> dPF[1][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          const f4 dp = dG1[o].v * sp1[o];
          dZ1[o].v = dG1[o].v * Pm[0][o].v * spp1[o];
          dPf[o] = to_frag<T>(dp);
          dPF[0][o] = to_frag<T>(transpose16(dPf[o], I).v);
        }
        Frag<T> w2t[FT][HT];
#pragma unroll
        for (int o = 0; o < FT; ++o)
#pragma unroll
          for (int c = 0; c < HT; ++c) w2t[o][c] = load_frag(W2t_ + (size_t)(16 * o) * FF, FF, hs + 16 * c);
        Tile dg2p[1][FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) dg2p[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, FT, HT>(dg2p, dPF, w2t);  // dP W2
#pragma unroll
        for (int o = 0; o < FT; ++o) sh.u.s.partB[wave][o][l] = dg2p[0][o].v;
      }
      __syncthreads();  // (4)

      // ---- B3: G2 backward (every wave), dX2, dZ1, dXK partials
#pragma unroll
      for (int o = 0; o < FT; ++o)
#pragma unroll
        for (int w = 0; w < NW; ++w) dG2[o].v += sh.u.s.partB[w][o][l];
      f4 dz2[FT], dtgt[FT];
      {
        float lw_i[FT], lb_i[FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          lw_i[o] = 0.f;
          lb_i[o] = 0.f;
        }
        ln2.backward(dG2, G2, lnw_tm, dz2, dtgt, lw_i, lb_i);
        if (wave == 0) {
#pragma unroll
          for (int o = 0; o < FT; ++o) {
            dlnw[o] += lw_i[o];
            dlnb[o] += lb_i[o];
          }
        }
      }
      Frag<T> dz2f[FT], dz2F[1][FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        dz2f[o] = to_frag<T>(dz2[o]);
        dz2F[0][o] = to_frag<T>(transpose16(dz2f[o], I).v);
      }
      Frag<T> dz1f[HT];
      {
        Tile dx2[1][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) dx2[0][o] = dX2[o];
        gemm<1, HT, FT>(dx2, dz2F, w2);  // + dZ2 W2^T
        Frag<T> dz1F[1][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          dZ1[o].v += dx2[0][o].v * sp1[o];
          dz1f[o] = to_frag<T>(dZ1[o].v);
          dz1F[0][o] = to_frag<T>(transpose16(dz1f[o], I).v);
        }
        Frag<T> w1[FT][HT];
#pragma unroll
        for (int o = 0; o < FT; ++o)
#pragma unroll
          for (int c = 0; c < HT; ++c) w1[o][c] = load_frag(W1_ + (size_t)(16 * o) * FF, FF, hs + 16 * c);
        Tile dxkp[1][FT];
#pragma unroll
        for (int o = 0; o < FT; ++o) dxkp[0][o].v = f4{0.f, 0.f, 0.f, 0.f};
        gemm<1, FT, HT>(dxkp, dz1F, w1);  // dZ1 W1^T
#pragma unroll
        for (int o = 0; o < FT; ++o) sh.u.s.partC[wave][o][l] = dxkp[0][o].v;
      }
      __syncthreads();  // (5)

      // ---- B4: dXK, dXV (wave 0); accumulate the state gradient
      if (wave == 0) {
        const Frag<T> dA1f = to_frag<T>(dA1);
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          Tile dxk;
          dxk.v = -dtgt[o];
#pragma unroll
          for (int w = 0; w < NW; ++w) dxk.v += sh.u.s.partC[w][o][l] + sh.u.s.partD[w][o][l];
          mma16(dxk.v, dA1f, xqTf[o]);  // + dA1^T XQ
          store_f4(DXK + xo, F, 16 * o, transpose16(to_frag<T>(dxk.v), I).v);
          store_f4(DXV + xo, F, 16 * o, transpose16(to_frag<T>(dtgt[o]), I).v);
        }
      }
#pragma unroll
      for (int q = 0; q < FT; ++q)
#pragma unroll
        for (int c = 0; c < HT; ++c) mma32(dW1[q][c].v, xqTf[q], xkTf[q], dz1bf[c], dz1f[c]);
#pragma unroll
      for (int c = 0; c < HT; ++c)
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          mma32(dW2[c][o].v, x2bf[c], dPf[c], dz2bf[o], g2f[o]);
          mma16(dW2[c][o].v, x2f[c], dz2f[o]);
        }
      // column sums in fp32: db1 += colsum(dZ1b + dZ1), db2 += colsum(dZ2b + dZ2)
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += dZ1[o].v[j];
        db1[o] += sum_col4(acc) + dz1b_cs[o];
      }
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += dz2[o][j];
        db2[o] += sum_col4(acc) + dz2b_cs[o];
      }
    }
  }

  // ---- outputs: gradient wrt the initial state, LN parameters
  {
    float* w1 = p.dW1 + (size_t)chain * F * FF;
    float* w2 = p.dW2 + (size_t)chain * FF * F;
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) store_tile(w1, FF, 16 * i, hs + 16 * o, dW1[i][o]);
#pragma unroll
    for (int i = 0; i < HT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) store_tile(w2, F, hs + 16 * i, 16 * o, dW2[i][o]);
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < HT; ++o) p.db1[(size_t)chain * FF + hs + 16 * o + n] = db1[o];
    }
  }
  if (wave == 0) {
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      const float w = sum_col4(dlnw[o]);
      const float b = sum_col4(dlnb[o]);
      if (g == 0) {
        p.db2[(size_t)chain * F + 16 * o + n] = db2[o];
        p.dln_w[(size_t)chain * F + 16 * o + n] = w;
        p.dln_b[(size_t)chain * F + 16 * o + n] = b;
      }
    }
  }
}

template <typename T, int FT, int NW>
static hipError_t launch_mlp_bwd_t(const MlpBwdParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((mlp_bwd_kernel<T, FT, NW>), dim3(p.B * p.H), dim3(64 * NW), 0, stream, p);
  return hipGetLastError();
}

template <typename T, int FT>
static hipError_t launch_mlp_bwd_f(const MlpBwdParams& p, hipStream_t stream) {
  switch (p.FF) {
    case 64: return launch_mlp_bwd_t<T, FT, 1>(p, stream);
    case 128: return launch_mlp_bwd_t<T, FT, 2>(p, stream);
    case 256: return launch_mlp_bwd_t<T, FT, 4>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_mlp_bwd(const MlpBwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_mlp_bwd_f<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_mlp_bwd_f<__bf16, 2>(p, stream);
  } else {
    if (p.F == 64) return launch_mlp_bwd_f<float, 4>(p, stream);
    if (p.F == 32) return launch_mlp_bwd_f<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

size_t mlp_bwd_slot_bytes(int F, int FF, int dtype) {
  const size_t t = dtype == TTT_DTYPE_BF16 ? 2 : 4;
  return 4 * (size_t)F * FF * t + (size_t)(FF + F) * sizeof(float);
}

}  // namespace ttt
