// TTT-Linear mini-batch forward on gfx950.
//
// One workgroup (one wavefront) owns one (batch, head) chain and keeps the
// fast weight W [F x F] and bias b [F] resident in registers (fp32, MFMA
// accumulator layout) across all NC sequential mini-batches.  Per mini-batch
// of K = 16 tokens (ops/ttt_linear.py:8-54, dual form with a full KxK eta):
//
//   Z1   = XK W + b                               (token-major tiles)
//   G    = ln_fused_l2_bwd(Z1, XV - XK)          (row reductions over F via DPP)
//   Zb^T = W^T XQ^T - G^T (eta o A + eta)^T + b   with A^T = XK XQ^T
//   out  = XQ + LN(Zb)                            (feature-major tiles, written
//                                                  4 contiguous elements per lane)
//   W   -= XK^T diag(eta[K-1]) G ;  b -= G^T eta[K-1]
//
// Inputs for mini-batch s+1 are loaded while mini-batch s computes.  The state
// entering mini-batch k*G is written to the checkpoint buffers
// (kernels/linear_forward.py:55-73 convention) and the final state to W_last.
// With a saved buffer, every mini-batch's G, normalised Z1 and Zb and their
// statistics go to its LinSavedSlot for the backward.
#include "ttt_buf.h"
#include "ttt_kernels.h"

namespace ttt {

template <typename T, int FT>
__global__ __launch_bounds__(64) void linear_fwd_kernel(LinearFwdParams p) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  const int chain = blockIdx.x;
  const int h = chain % p.H;
  const int NC = p.NC;
  const int l = lane_id(), g = l >> 4, n = l & 15;

  const T* __restrict__ XQ = static_cast<const T*>(p.XQ) + (size_t)chain * NC * K * F;
  const T* __restrict__ XK = static_cast<const T*>(p.XK) + (size_t)chain * NC * K * F;
  const T* __restrict__ XV = static_cast<const T*>(p.XV) + (size_t)chain * NC * K * F;
  const T* __restrict__ ETA = static_cast<const T*>(p.eta) + (size_t)chain * NC * K * K;
  T* __restrict__ OUT = static_cast<T*>(p.out) + (size_t)chain * NC * K * F;
  using Slot = LinSavedSlot<F>;
  // Saved values go through a buffer resource whose size is zero when there is
  // no saved buffer: the stores are then dropped by the range check, and being
  // unconditional they keep the wait counts before the next mini-batch's
  // prefetched inputs exact.
  const rsrc_t SV = p.saved ? make_rsrc(static_cast<char*>(p.saved) + (size_t)chain * NC * Slot::BYTES,
                                        (unsigned)(NC * Slot::BYTES))
                            : make_rsrc(p.out, 0u);

  __shared__ float b_lds[F];

  Tile W[FT][FT];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < FT; ++o) W[i][o] = load_tile(p.W_init + (size_t)chain * F * F, F, 16 * i, 16 * o);
  float b_tm[FT];
#pragma unroll
  for (int o = 0; o < FT; ++o) b_tm[o] = p.b_init[(size_t)chain * F + 16 * o + n];
  for (int f = l; f < F; f += 64) b_lds[f] = p.b_init[(size_t)chain * F + f];

  float lnw_tm[FT], lnb_tm[FT];
  f4 lnw_fm[FT], lnb_fm[FT];
#pragma unroll
  for (int o = 0; o < FT; ++o) {
    lnw_tm[o] = p.ln_w[h * F + 16 * o + n];
    lnb_tm[o] = p.ln_b[h * F + 16 * o + n];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lnw_fm[o][j] = p.ln_w[h * F + 16 * o + 4 * g + j];
      lnb_fm[o][j] = p.ln_b[h * F + 16 * o + 4 * g + j];
    }
  }
  const float eps = p.eps;
  const float invF = 1.0f / F;
  const Frag<T> I = identity_frag<T>();

  // prefetched inputs of the next mini-batch
  Frag<T> nq[1][FT], nk[1][FT], nv[1][FT];
  Frag<T> n_etaT, n_e;  // raw: converted where used, so the prefetch is not waited for
  auto load_step = [&](int s) {
    const T* q = XQ + (size_t)s * K * F;
    const T* k = XK + (size_t)s * K * F;
    const T* v = XV + (size_t)s * K * F;
#pragma unroll
    for (int c = 0; c < FT; ++c) {
      nq[0][c] = load_frag(q, F, 16 * c);
      nk[0][c] = load_frag(k, F, 16 * c);
      nv[0][c] = load_frag(v, F, 16 * c);
    }
    const T* e = ETA + (size_t)s * K * K;
    n_etaT = load_frag(e, K, 0);            // lane (g,n): eta[n][4g+j]
    n_e = load_frag(e + (K - 1) * K, 0, 0);  // lane (g,*): eta[K-1][4g+j]
  };
  load_step(0);
  // Retire the first loads before the loop: with them pending on entry the
  // wait-count pass cannot order them against the loop's own loads and stores
  // and waits for every outstanding access in each iteration.
  __builtin_amdgcn_s_waitcnt(0);

  for (int s = 0; s < NC; ++s) {
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

    Frag<T> xq[1][FT], xk[1][FT], xv[1][FT];
#pragma unroll
    for (int c = 0; c < FT; ++c) {
      xq[0][c] = nq[0][c];
      xk[0][c] = nk[0][c];
      xv[0][c] = nv[0][c];
    }
    const Frag<T> etaT_raw = n_etaT, e_raw = n_e;
    if (s + 1 < NC) load_step(s + 1);

    // W as operand frags: Wf[o][i] (free = f_out block o, contraction = f_in block i)
    Frag<T> Wf[FT][FT];
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) Wf[o][i] = to_frag<T>(W[i][o].v);

    // Z1 = XK W + b (token-major)
    Tile z1[1][FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) z1[0][o].v = f4{b_tm[o], b_tm[o], b_tm[o], b_tm[o]};
    gemm<1, FT, FT>(z1, xk, Wf);

    // Zb^T = W^T XQ^T (feature-major), dual and bias terms added below
    Tile zb[FT][1];
#pragma unroll
    for (int o = 0; o < FT; ++o) zb[o][0].v = f4{0.f, 0.f, 0.f, 0.f};
    gemm<FT, 1, FT>(zb, Wf, xq);

    // A^T = XK XQ^T : C layout [t_k x t_q]
    Tile at[1][1];
    at[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
    gemm<1, 1, FT>(at, xk, xq);

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
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) G[o].v[j] = (gx[o][j] - s1[j] - xh[o][j] * s2[j]) * rstd[j];
    const int sv = s * Slot::BYTES;
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      bstore_frag<float>(SV, 16 * l + 1024 * o, sv + Slot::G, Frag<float>{G[o].v});
      bstore_frag<float>(SV, 16 * l + 1024 * o, sv + Slot::XH, Frag<float>{xh[o]});
    }
    // per-row values: the 16 lanes of a group store the same 4 rows
    bstore_frag<float>(SV, 16 * g, sv + Slot::RSTD, Frag<float>{rstd});
    bstore_frag<float>(SV, 16 * g, sv + Slot::CC, Frag<float>{s2});

    // ---- readout: Zb^T -= G^T (eta o A + eta)^T ; + b
    {
      f4 mt;
      const f4 etaT = frag_to_f4(etaT_raw);
#pragma unroll
      for (int j = 0; j < 4; ++j) mt[j] = etaT[j] * at[0][0].v[j] + etaT[j];
      const Frag<T> mtf = to_frag<T>(mt);
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        const Frag<T> gneg = to_frag<T>(-G[o].v);
        mma16(zb[o][0].v, gneg, mtf);
#pragma unroll
        for (int j = 0; j < 4; ++j) zb[o][0].v[j] += b_lds[16 * o + 4 * g + j];
      }
    }

    // ---- state update: W -= XK^T diag(e) G ; b -= G^T e
    {
      const f4 e = frag_to_f4(e_raw);
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
        if (g == 0) b_lds[16 * o + n] = b_tm[o];
      }
    }

    // ---- LN over features of each token (token n lives in lanes n, n+16, n+32, n+48)
    {
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
}

template <typename T, int FT>
static hipError_t launch_fwd(const LinearFwdParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((linear_fwd_kernel<T, FT>), dim3(p.B * p.H), dim3(64), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_linear_fwd(const LinearFwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_fwd<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_fwd<__bf16, 2>(p, stream);
  } else {
    if (p.F == 64) return launch_fwd<float, 4>(p, stream);
    if (p.F == 32) return launch_fwd<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
