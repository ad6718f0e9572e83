// TTT-Linear mini-batch forward on gfx950, fp32 activations (16-bit
// activations run the row-split kernel of ttt_linear_fwd_rows.hip).
//
// One workgroup of two wavefronts per (batch, head) chain.  Per mini-batch of
// K = 16 tokens (ops/ttt_linear.py:8-54, dual form with a full KxK eta):
//
//   Z1   = XK W + b                               (token-major tiles)
//   G    = ln_fused_l2_bwd(Z1, XV - XK)          (row reductions over F via DPP)
//   W   -= XK^T diag(eta[K-1]) G ;  b -= G^T eta[K-1]
//   Zb^T = W^T XQ^T - G^T (eta o A + eta)^T + b   with A^T = XK XQ^T, W and b
//                                                  the state entering the mini-batch
//   out  = XQ + LN(Zb)                            (feature-major tiles, written
//                                                  4 contiguous elements per lane)
//
// Only the first three lines carry the recurrence.  Wave 0 (the recurrence)
// keeps W [F x F] and b resident in registers (fp32, MFMA accumulator layout)
// across all NC mini-batches and, per mini-batch, hands the readout what it
// needs of the state and the inner-loss gradient through LDS: W's operand
// frags (converted for Z1 anyway), -G as frags and b.  Wave 1 (the readout)
// forms Zb and the output of mini-batch s while wave 0 already runs s+1; the
// handoff is double-buffered by mini-batch parity with one barrier per
// mini-batch, so wave 0's critical path is Z1, the LayerNorm gradient and the
// update alone.
//
// Inputs for mini-batch s+1 are loaded while mini-batch s computes.  The state
// entering mini-batch k*G is written to the checkpoint buffers
// (kernels/linear_forward.py:55-73 convention) and the final state to W_last.
// With a saved buffer, every mini-batch's G, normalised Z1 and Zb and their
// statistics go to its LinSavedSlot for the backward.
#include <type_traits>

#include "ttt_buf.h"
#include "ttt_eta.h"
#include "ttt_kernels.h"

namespace ttt {

template <typename T, int FT> struct LinFwdHandoff {
  typename FragT<T>::type wf[FT * FT][64];  // W operand frags Wf[o][i] (free = f_out block o, k = f_in block i)
  typename FragT<T>::type gneg[FT][64];     // -G token-major tiles as frags
  float b[16 * FT];                         // b entering the mini-batch
};

template <typename T, int FT, bool LR, typename ET = T>
__global__ __launch_bounds__(128) void linear_fwd_kernel(LinearFwdParams p) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  const int chain = blockIdx.x;
  const int h = chain % p.H;
  const int NC = p.NC;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), g = l >> 4, n = l & 15;

  const T* __restrict__ XQ = static_cast<const T*>(p.XQ) + (size_t)chain * NC * K * F;
  const T* __restrict__ XK = static_cast<const T*>(p.XK) + (size_t)chain * NC * K * F;
  const T* __restrict__ XV = static_cast<const T*>(p.XV) + (size_t)chain * NC * K * F;
  // eta: dense [NC][K][K] blocks of ET, or (LR) the learning rates lr [NC][K]
  // fp32 that the eta rule expands on chip; held raw until used
  const ET* __restrict__ ETA = LR ? nullptr : static_cast<const ET*>(p.eta) + (size_t)chain * NC * K * K;
  const float* __restrict__ LRP = LR ? static_cast<const float*>(p.eta) + (size_t)chain * NC * K : nullptr;
  using ERaw = std::conditional_t<LR, f4, Frag<ET>>;
  const int eta_rule = p.eta_rule;
  T* __restrict__ OUT = static_cast<T*>(p.out) + (size_t)chain * NC * K * F;
  using Slot = LinSavedSlot<F>;
  // Saved values go through a buffer resource whose size is zero when there is
  // no saved buffer: the stores are then dropped by the range check, and being
  // unconditional they keep the wait counts before the next mini-batch's
  // prefetched inputs exact.
  const rsrc_t SV = p.saved ? make_rsrc(static_cast<char*>(p.saved) + (size_t)chain * NC * Slot::BYTES,
                                        (unsigned)(NC * Slot::BYTES))
                            : make_rsrc(p.out, 0u);
  __shared__ LinFwdHandoff<T, FT> hand[2];
  const float eps = p.eps;
  const float invF = 1.0f / F;
  const Frag<T> I = identity_frag<T>();

  if (wave == 0) {
    // ================================================================ recurrence
    Tile W[FT][FT];
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) W[i][o] = load_tile(p.W_init + (size_t)chain * F * F, F, 16 * i, 16 * o);
    float b_tm[FT], lnw_tm[FT], lnb_tm[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      b_tm[o] = p.b_init[(size_t)chain * F + 16 * o + n];
      lnw_tm[o] = p.ln_w[h * F + 16 * o + n];
      lnb_tm[o] = p.ln_b[h * F + 16 * o + n];
    }

    // prefetched inputs of the next mini-batch (raw: converted where used, so
    // the prefetch is not waited for early)
    Frag<T> nk[1][FT], nv[1][FT];
    ERaw n_e;
    auto load_step = [&](int s) {
      const T* k = XK + (size_t)s * K * F;
      const T* v = XV + (size_t)s * K * F;
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        nk[0][c] = load_frag(k, F, 16 * c);
        nv[0][c] = load_frag(v, F, 16 * c);
      }
      if constexpr (LR)
        n_e = *reinterpret_cast<const f4*>(LRP + (size_t)s * K + 4 * g);  // lane (g,*): lr[4g+j]
      else
        n_e = load_frag(ETA + (size_t)s * K * K + (K - 1) * K, 0, 0);  // lane (g,*): eta[K-1][4g+j]
    };
    load_step(0);
    // Retire the first loads before the loop: with them pending on entry the
    // wait-count pass cannot order them against the loop's own loads and stores
    // and waits for every outstanding access in each iteration.
    __builtin_amdgcn_s_waitcnt(0);

    for (int s = 0; s < NC; ++s) {
      // the state stays in the accumulator registers (the MFMA update's own)
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) asm volatile("" : "+a"(W[i][o].v));
      if (p.W_ckpt != nullptr && (s % p.G) == 0) {
        const int kk = s / p.G;
        float* wc = p.W_ckpt + ((size_t)chain * p.NK + kk) * F * F;
#pragma unroll
        for (int i = 0; i < FT; ++i)
#pragma unroll
          for (int o = 0; o < FT; ++o) store_tile(wc, F, 16 * i, 16 * o, W[i][o]);
        if (g == 0) {
#pragma unroll
          for (int o = 0; o < FT; ++o) p.b_ckpt[((size_t)chain * p.NK + kk) * F + 16 * o + n] = b_tm[o];
        }
      }
      Frag<T> xk[1][FT], xv[1][FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        xk[0][c] = nk[0][c];
        xv[0][c] = nv[0][c];
      }
      const ERaw e_raw = n_e;
      if (s + 1 < NC) load_step(s + 1);
      LinFwdHandoff<T, FT>& hs = hand[s & 1];

      // W as operand frags, handed to the readout with b
      Frag<T> Wf[FT][FT];
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          Wf[o][i] = to_frag<T>(W[i][o].v);
          hs.wf[o * FT + i][l] = Wf[o][i].v;
        }
      if (g == 0) {
#pragma unroll
        for (int o = 0; o < FT; ++o) hs.b[16 * o + n] = b_tm[o];
      }

      // Z1 = XK W + b (token-major)
      Tile z1[1][FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) z1[0][o].v = f4{b_tm[o], b_tm[o], b_tm[o], b_tm[o]};
      gemm<1, FT, FT>(z1, xk, Wf);

      // token-major XK and XV (exact transposes)
      Tile xkT[FT], xvT[FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        xkT[c] = transpose16(xk[0][c], I);
        xvT[c] = transpose16(xv[0][c], I);
      }

      // ---- ln_fused_l2_bwd on Z1 rows (row t = 4g + j spans 16 lanes x FT tiles)
      f4 mu, rstd;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float sacc = 0.f;
#pragma unroll
        for (int o = 0; o < FT; ++o) sacc += z1[0][o].v[j];
        mu[j] = sum_row16(sacc) * invF;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float sacc = 0.f;
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          const float d = z1[0][o].v[j] - mu[j];
          sacc += d * d;
        }
        rstd[j] = rsqrt_f(sum_row16(sacc) * invF + eps);
      }
      f4 xh[FT], gx[FT];
      f4 s1 = f4{0.f, 0.f, 0.f, 0.f}, s2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int o = 0; o < FT; ++o)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xh[o][j] = (z1[0][o].v[j] - mu[j]) * rstd[j];
          const float tgt = xvT[o].v[j] - xkT[o].v[j];
          gx[o][j] = (lnw_tm[o] * xh[o][j] + lnb_tm[o] - tgt) * lnw_tm[o];
          s1[j] += gx[o][j];
          s2[j] += gx[o][j] * xh[o][j];
        }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s1[j] = sum_row16(s1[j]) * invF;
        s2[j] = sum_row16(s2[j]) * invF;
      }
      Tile G[FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
#pragma unroll
        for (int j = 0; j < 4; ++j) G[o].v[j] = (gx[o][j] - s1[j] - xh[o][j] * s2[j]) * rstd[j];
        hs.gneg[o][l] = to_frag<T>(-G[o].v).v;
      }
      const int sv = s * Slot::BYTES;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        bstore_frag<float>(SV, 16 * l + 1024 * o, sv + Slot::G, Frag<float>{G[o].v});
        bstore_frag<float>(SV, 16 * l + 1024 * o, sv + Slot::XH, Frag<float>{xh[o]});
      }
      // per-row values: the 16 lanes of a group store the same 4 rows
      bstore_frag<float>(SV, 16 * g, sv + Slot::RSTD, Frag<float>{rstd});
      bstore_frag<float>(SV, 16 * g, sv + Slot::CC, Frag<float>{s2});

      // ---- state update: W -= XK^T diag(e) G ; b -= G^T e
      {
        f4 e;
        if constexpr (LR)
          e = eta_lastrow_from_lr(e_raw);
        else
          e = frag_to_f4(e_raw);
        Frag<T> xkf[FT], ge[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          xkf[c] = to_frag<T>(xkT[c].v);
          f4 v;
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = -e[j] * G[c].v[j];
          ge[c] = to_frag<T>(v);
        }
#pragma unroll
        for (int i = 0; i < FT; ++i)
#pragma unroll
          for (int o = 0; o < FT; ++o) mma16(W[i][o].v, xkf[i], ge[o]);
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          float acc = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc += e[j] * G[o].v[j];
          b_tm[o] -= sum_col4(acc);
        }
      }
      __syncthreads();  // mini-batch s handed over
    }

    if (p.W_last != nullptr) {
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) store_tile(p.W_last + (size_t)chain * F * F, F, 16 * i, 16 * o, W[i][o]);
      if (g == 0) {
#pragma unroll
        for (int o = 0; o < FT; ++o) p.b_last[(size_t)chain * F + 16 * o + n] = b_tm[o];
      }
    }
  } else {
    // ================================================================ readout
    f4 lnw_fm[FT], lnb_fm[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lnw_fm[o][j] = p.ln_w[h * F + 16 * o + 4 * g + j];
        lnb_fm[o][j] = p.ln_b[h * F + 16 * o + 4 * g + j];
      }
    Frag<T> nq[1][FT], nk[1][FT];
    ERaw n_etaT;
    auto load_step = [&](int s) {
      const T* q = XQ + (size_t)s * K * F;
      const T* k = XK + (size_t)s * K * F;
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        nq[0][c] = load_frag(q, F, 16 * c);
        nk[0][c] = load_frag(k, F, 16 * c);
      }
      if constexpr (LR)
        n_etaT = *reinterpret_cast<const f4*>(LRP + (size_t)s * K + 4 * g);  // lane (g,*): lr[4g+j]
      else
        n_etaT = load_frag(ETA + (size_t)s * K * K, K, 0);  // lane (g,n): eta[n][4g+j]
    };
    load_step(0);
    __builtin_amdgcn_s_waitcnt(0);

    for (int s = 0; s < NC; ++s) {
      Frag<T> xq[1][FT], xk[1][FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        xq[0][c] = nq[0][c];
        xk[0][c] = nk[0][c];
      }
      const ERaw etaT_raw = n_etaT;
      if (s + 1 < NC) load_step(s + 1);
      __syncthreads();  // mini-batch s handed over
      const LinFwdHandoff<T, FT>& hs = hand[s & 1];

      // Zb^T = W^T XQ^T (feature-major) - G^T (eta o A + eta)^T + b
      Frag<T> Wf[FT][FT];
#pragma unroll
      for (int o = 0; o < FT; ++o)
#pragma unroll
        for (int i = 0; i < FT; ++i) Wf[o][i].v = hs.wf[o * FT + i][l];
      Tile zb[FT][1];
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const f4 bo = *reinterpret_cast<const f4*>(&hs.b[16 * o + 4 * g]);
        zb[o][0].v = bo;
      }
      gemm<FT, 1, FT>(zb, Wf, xq);
      Tile at[1][1];  // A^T = XK XQ^T : C layout [t_k x t_q]
      at[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      gemm<1, 1, FT>(at, xk, xq);
      {
        f4 mt;
        f4 etaT;
        if constexpr (LR)
          etaT = eta_rowfrag_from_lr(eta_rule, etaT_raw);
        else
          etaT = frag_to_f4(etaT_raw);
#pragma unroll
        for (int j = 0; j < 4; ++j) mt[j] = etaT[j] * at[0][0].v[j] + etaT[j];
        const Frag<T> mtf = to_frag<T>(mt);
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          Frag<T> gneg;
          gneg.v = hs.gneg[o][l];
          mma16(zb[o][0].v, gneg, mtf);
        }
      }

      // ---- LN over features of each token (token n lives in lanes n, n+16, n+32, n+48)
      const int sv = s * Slot::BYTES;
      float sacc = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o)
#pragma unroll
        for (int j = 0; j < 4; ++j) sacc += zb[o][0].v[j];
      const float m = sum_col4(sacc) * invF;
      float vacc = 0.f;
#pragma unroll
      for (int o = 0; o < FT; ++o)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float d = zb[o][0].v[j] - m;
          vacc += d * d;
        }
      const float rs = rsqrt_f(sum_col4(vacc) * invF + eps);
      T* o_s = OUT + (size_t)s * K * F;
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const f4 q = frag_to_f4(xq[0][o]);
        f4 xhb, y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xhb[j] = (zb[o][0].v[j] - m) * rs;
          y[j] = q[j] + lnw_fm[o][j] * xhb[j] + lnb_fm[o][j];
        }
        store_f4(o_s, F, 16 * o, y);
        bstore_frag<float>(SV, 16 * l + 1024 * o, sv + Slot::XHB, Frag<float>{xhb});
      }
      bstore_f32(SV, 4 * n, sv + Slot::RSB, rs);  // per token: the 4 lanes of token n agree
    }
  }
}

template <typename T, int FT>
static hipError_t launch_fwd(const LinearFwdParams& p, hipStream_t stream) {
  if (p.eta_rule == TTT_ETA_DENSE)
    hipLaunchKernelGGL((linear_fwd_kernel<T, FT, false>), dim3(p.B * p.H), dim3(128), 0, stream, p);
  else if (p.eta_rule == TTT_ETA_DENSE_F32)
    hipLaunchKernelGGL((linear_fwd_kernel<T, FT, false, float>), dim3(p.B * p.H), dim3(128), 0, stream, p);
  else
    hipLaunchKernelGGL((linear_fwd_kernel<T, FT, true>), dim3(p.B * p.H), dim3(128), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_linear_fwd(const LinearFwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16 || dtype == TTT_DTYPE_F16) {
    return launch_linear_fwd_rows(p, dtype, stream);
  } else {
    if (p.F == 64) return launch_fwd<float, 4>(p, stream);
    if (p.F == 32) return launch_fwd<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
