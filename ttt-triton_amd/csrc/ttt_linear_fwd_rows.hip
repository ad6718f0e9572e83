// TTT-Linear mini-batch forward on gfx950, 16-bit activations (bf16, fp16):
// the recurrence split by token rows.
//
// Per mini-batch of K = 16 tokens (ops/ttt_linear.py:8-54, dual form with a
// full KxK eta), as the fp32 kernel of ttt_linear_fwd.hip computes it:
//
//   Z1   = XK W + b,  G = ln_fused_l2_bwd(Z1, XV - XK)
//   W   -= XK^T diag(eta[K-1]) G ;  b -= G^T eta[K-1]
//   Zb   = XQ W - (eta o XQ XK^T + eta) G + b   (W, b entering the mini-batch)
//   out  = XQ + LN(Zb)
//
// Four wavefronts per chain.  The state update enters the next mini-batch's
// Z1 as a 16 x 16 correction (the look-ahead form):
//
//   Z1_s = P_s + M_{s-1} (-G_{s-1}) + 1 b_{s-1}^T,   P_s = XK_s W_{s-1},
//   M_{s-1} = (XK_s XK_{s-1}^T + 1 1^T) diag(e_{s-1}),
//
// so G_{s-1} is all that mini-batch s waits for.  Everything runs
// feature-major (Z1^T = W^T XK^T: W's accumulator tiles and XK's loaded frags
// are the operands as they stand).
//   R0, R1  the chain, split by token rows: Rw forms the correction for all
//           16 tokens (4 MFMAs), packs its tokens 8w..8w+7 into all 64 lanes
//           (lane (g, n) holds token (n & 7) + 8w, features 4g..4g+3 of tiles
//           2p + (n >> 3): a row sum is in-lane adds, one row_ror:8 and two
//           lane swaps), adds P_s and b_{s-1}, and forms G for its tokens;
//   S       the state: W and b, the update with G_{s-1}, W_s's operand frags,
//           P_{s+1} (handed over in each R wave's packed lane order), M_s,
//           the checkpoints, and the saved slot's G;
//   O       the readout of mini-batch s-1, and the saved slot's XH and row
//           values.
// G goes through LDS as 16-bit rows (-G, and -(e o G) for the update) that
// every consumer reads back with ds_read_b64_tr_b16, which is the transpose
// the token-major operands need, and as fp32 rows with XH for S and O (the
// saved slot's token-major tiles, written as 16-byte rows).  XK is loaded
// from HBM by S alone, which stages it in LDS as 16-bit rows for the other
// three waves (R's rows, O's frags, S's own transposing read): the waves
// share the CU's memory pipeline, and the shared XK took the kernel from
// 199.6 to 186 us.  One barrier per
// mini-batch; every handoff double-buffered by parity.  The products keep
// their accumulators in VGPRs (this file is compiled with
// -amdgpu-mfma-vgpr-form, so converting W into operand frags reads no
// accumulator registers).
//
// Against the two-wave kernel (one recurrence wave carrying the whole
// LayerNorm, the update and W's conversion): 200 against 224 us at B16 H12
// T2048 F64 bf16; the waves share the CU's memory pipelines, and timing
// copies with O or S idle ran at 161 and 150 us.
#include <type_traits>

#include "ttt_buf.h"
#include "ttt_eta.h"
#include "ttt_kernels.h"

namespace ttt {

template <typename T, int FT> struct LinRowsPar {
  typename FragT<T>::type wf[FT * FT][64];  // W_s operand frags [o * FT + i]
  float b[16 * FT];                         // b_s
  u2v gneg[FT][64];                         // -G_s: tile o, token t, features 16 o + 4 g.. at grow_put(o, t, g)
  u2v geta[FT][64];                         // -(e_s o G_s), same places
  f4 pp[2][FT / 2][64];                     // [w]: P_{s+1}^T in R_w's packed lane order
  u2v mt[64];                               // M_s^T operand frag
  float gx[2][FT][16][20];                  // fp32 G_s, XH_s: [tile][token][feature % 16] (rows padded)
  float rc[2][16];                          // rstd_s, c_s per token
};
template <typename T, int FT> struct LinRowsShared {
  LinRowsPar<T, FT> par[2];
  u2v xkt[3][FT][64];                       // XK_s in slot s % 3 as 16-bit rows (grow_put per tile):
                                            // S writes XK_{s+1} while mini-batch s runs; R reads XK_s's
                                            // rows, O XK_{s-1}'s frags, S XK_{s-1} transposed
};

typedef short s4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4v lds_s4v;
// ds_read_b64_tr_b16: the 16 lanes of group g' each supply the address of one
// 4-element row M[i]; lane i receives M[4k + i/4][i%4] for k = 0..3.  With row
// i of group g' = elements X[4g' + i/4][4 (i%4) .. +3] of a 16 x 16 matrix X
// written by rows, lane (g', i) receives X[4g' + k][i]: X's C-layout frag
// from its row-layout frag.
template <typename T> __device__ __forceinline__ Frag<T> lds_read_tr(const u2v* p) {
  const s4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v*)(const_cast<u2v*>(p)));
  Frag<T> f;
  f.v = __builtin_bit_cast(typename FragT<T>::type, r);
  return f;
}
template <typename T> __device__ __forceinline__ u2v frag_bits(Frag<T> f) { return __builtin_bit_cast(u2v, f.v); }
template <typename T> __device__ __forceinline__ Frag<T> bits_frag(u2v v) {
  Frag<T> f;
  f.v = __builtin_bit_cast(typename FragT<T>::type, v);
  return f;
}
// the 16-bit tile rows' places (ttt_lds_layout.h: conflict-free row writes,
// transposing reads)
using lds::grow_get;
using lds::grow_put;

// lane (g, n) of R_w's packed form: own value of tile 2p + w where n >> 3 == w,
// else tile 2p + 1 - w from lane n ^ 8 (row_ror:8 within the 16-lane row)
template <int W> __device__ __forceinline__ f4 pack_rows(f4 t0, f4 t1) {
  f4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int own = __builtin_bit_cast(int, W == 0 ? t0[j] : t1[j]);
    const int oth = __builtin_bit_cast(int, W == 0 ? t1[j] : t0[j]);
    r[j] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(own, oth, 0x128, 0xF, W == 0 ? 0xC : 0x3, false));
  }
  return r;
}

// ---- R_w: the inner-loss LayerNorm gradient of tokens 8w..8w+7
template <typename T, int FT, bool LR, typename ET, int W>
__device__ __forceinline__ void linear_rows_chain(const LinearFwdParams& p, LinRowsShared<T, FT>& sh) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  constexpr int PP = FT / 2;
  const int chain = blockIdx.x;
  const int h = chain % p.H;
  const int NC = p.NC;
  const int l = lane_id(), g = l >> 4, n = l & 15, hi = n >> 3;
  const int t = (n & 7) + 8 * W;  // this lane's token in the packed form
  const T* __restrict__ XV = static_cast<const T*>(p.XV) + (size_t)chain * NC * K * F;
  const ET* __restrict__ ETA = LR ? nullptr : static_cast<const ET*>(p.eta) + (size_t)chain * NC * K * K;
  const float* __restrict__ LRP = LR ? static_cast<const float*>(p.eta) + (size_t)chain * NC * K : nullptr;
  const float eps = p.eps;
  const float invF = 1.0f / F;
  using VT = typename FragT<T>::type;
  using EOne = std::conditional_t<LR, float, ET>;

  f4 lnw_pk[PP], lnb_pk[PP];
#pragma unroll
  for (int q = 0; q < PP; ++q) {
    const int f0 = 16 * (2 * q + hi) + 4 * g;
    lnw_pk[q] = *reinterpret_cast<const f4*>(p.ln_w + h * F + f0);
    lnb_pk[q] = *reinterpret_cast<const f4*>(p.ln_b + h * F + f0);
  }
  // XV and XK of token t (packed) and eta[K-1][t] of the next mini-batch, raw
  VT tv_n[PP];
  EOne et_n;
  auto load_row = [&](int s) {
    const T* v = XV + (size_t)s * K * F + t * F;
#pragma unroll
    for (int q = 0; q < PP; ++q) tv_n[q] = *reinterpret_cast<const VT*>(v + 16 * (2 * q + hi) + 4 * g);
    if constexpr (LR)
      et_n = LRP[(size_t)s * K + t];
    else
      et_n = ETA[(size_t)s * K * K + (K - 1) * K + t];
  };
  load_row(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // prologue

  for (int s = 0; s < NC; ++s) {
    VT tv[PP], tk[PP];
#pragma unroll
    for (int q = 0; q < PP; ++q) {
      tv[q] = tv_n[q];
      tk[q] = __builtin_bit_cast(VT, sh.xkt[s % 3][2 * q + hi][grow_put(2 * q + hi, t, g)]);  // XK_s, token t
    }
    const EOne et = et_n;
    if (s + 1 < NC) load_row(s + 1);
    LinRowsPar<T, FT>& cur = sh.par[s & 1];
    const LinRowsPar<T, FT>& prv = sh.par[(s + 1) & 1];

    // Z1_s^T = P_s^T + (-G_{s-1})^T M_{s-1}^T + b_{s-1}, this wave's tokens
    const Frag<T> Mt = bits_frag<T>(prv.mt[l]);
    Tile c[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      c[o].v = f4{0.f, 0.f, 0.f, 0.f};
      mma16(c[o].v, lds_read_tr<T>(&prv.gneg[o][grow_get(o, l)]), Mt);
    }
    f4 z[PP];
#pragma unroll
    for (int q = 0; q < PP; ++q)
      z[q] = pack_rows<W>(c[2 * q].v, c[2 * q + 1].v) + prv.pp[W][q][l] +
             *reinterpret_cast<const f4*>(&prv.b[16 * (2 * q + hi) + 4 * g]);

    // ---- ln_fused_l2_bwd on token t's row (4 PP values per lane)
    auto rsum = [](float v) { return sum_col4(v + dpp<0x128>(v)); };
    float sacc = z[0][0];
#pragma unroll
    for (int q = 0; q < PP; ++q)
#pragma unroll
      for (int j = (q == 0 ? 1 : 0); j < 4; ++j) sacc += z[q][j];
    const float mu = rsum(sacc) * invF;
    f4 d[PP];
#pragma unroll
    for (int q = 0; q < PP; ++q) d[q] = z[q] - mu;
    float vacc = d[0][0] * d[0][0];
#pragma unroll
    for (int q = 0; q < PP; ++q)
#pragma unroll
      for (int j = (q == 0 ? 1 : 0); j < 4; ++j) vacc += d[q][j] * d[q][j];
    const float rstd = rsqrt_f(rsum(vacc) * invF + eps);
    f4 xh[PP], gx[PP];
#pragma unroll
    for (int q = 0; q < PP; ++q) {
      const f4 tgt = frag_to_f4(Frag<T>{tv[q]}) - frag_to_f4(Frag<T>{tk[q]});
      xh[q] = d[q] * rstd;
      gx[q] = (lnw_pk[q] * xh[q] + lnb_pk[q] - tgt) * lnw_pk[q];
    }
    float s1 = gx[0][0], s2 = gx[0][0] * xh[0][0];
#pragma unroll
    for (int q = 0; q < PP; ++q)
#pragma unroll
      for (int j = (q == 0 ? 1 : 0); j < 4; ++j) {
        s1 += gx[q][j];
        s2 += gx[q][j] * xh[q][j];
      }
    s1 = rsum(s1) * invF;
    s2 = rsum(s2) * invF;
    const float e_t = LR ? (float)et * (1.0f / K) : (float)et;
#pragma unroll
    for (int q = 0; q < PP; ++q) {
      const f4 G = (gx[q] - s1 - xh[q] * s2) * rstd;
      cur.gneg[2 * q + hi][grow_put(2 * q + hi, t, g)] = frag_bits(to_frag<T>(-G));
      cur.geta[2 * q + hi][grow_put(2 * q + hi, t, g)] = frag_bits(to_frag<T>(-(e_t * G)));
      *reinterpret_cast<f4*>(&cur.gx[0][2 * q + hi][t][4 * g]) = G;
      *reinterpret_cast<f4*>(&cur.gx[1][2 * q + hi][t][4 * g]) = xh[q];
    }
    if (g == 0 && hi == 0) {
      cur.rc[0][t] = rstd;
      cur.rc[1][t] = s2;
    }
    __syncthreads();  // mini-batch s handed over
  }
}

// ---- S: the state
template <typename T, int FT, bool LR, typename ET>
__device__ __forceinline__ void linear_rows_state(const LinearFwdParams& p, LinRowsShared<T, FT>& sh) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  const int chain = blockIdx.x;
  const int NC = p.NC;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  const T* __restrict__ XK = static_cast<const T*>(p.XK) + (size_t)chain * NC * K * F;
  const ET* __restrict__ ETA = LR ? nullptr : static_cast<const ET*>(p.eta) + (size_t)chain * NC * K * K;
  const float* __restrict__ LRP = LR ? static_cast<const float*>(p.eta) + (size_t)chain * NC * K : nullptr;
  using Slot = LinSavedSlot<F>;
  const rsrc_t SV = p.saved ? make_rsrc(static_cast<char*>(p.saved) + (size_t)chain * NC * Slot::BYTES,
                                        (unsigned)(NC * Slot::BYTES))
                            : make_rsrc(p.out, 0u);
  using VT = typename FragT<T>::type;
  using ERow = std::conditional_t<LR, f4, Frag<ET>>;

  Tile W[FT][FT];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < FT; ++o) W[i][o] = load_tile(p.W_init + (size_t)chain * F * F, F, 16 * i, 16 * o);
  float bn[FT];  // b[16 o + n]
#pragma unroll
  for (int o = 0; o < FT; ++o) bn[o] = p.b_init[(size_t)chain * F + 16 * o + n];

  Frag<T> xk_cur[FT], xk_nxt[FT], xk_pf[FT];
  ERow er_n;
  auto load_xk = [&](Frag<T>(&dst)[FT], int s) {
    const T* k = XK + (size_t)s * K * F;
#pragma unroll
    for (int c = 0; c < FT; ++c) dst[c] = load_frag(k, F, 16 * c);
  };
  auto load_e = [&](int s) {
    if constexpr (LR)
      er_n = *reinterpret_cast<const f4*>(LRP + (size_t)s * K + 4 * g);
    else
      er_n = load_frag(ETA + (size_t)s * K * K + (K - 1) * K, 0, 0);  // lane (g,*): eta[K-1][4g+j]
  };
  auto e_of = [](ERow r) {
    if constexpr (LR)
      return eta_lastrow_from_lr(r);
    else
      return frag_to_f4(r);
  };
  load_xk(xk_cur, 0);
  load_xk(xk_nxt, NC > 1 ? 1 : 0);
  load_e(0);
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int c = 0; c < FT; ++c) xk_pf[c] = xk_nxt[c];  // finite operands for the unused look-ahead past the end
  f4 e_prev = f4{0.f, 0.f, 0.f, 0.f};

  // P_s^T (all block rows, all tokens) into both R waves' packed lane order
  auto put_p = [&](LinRowsPar<T, FT>& dst, const Frag<T>(&Wf)[FT][FT], const Frag<T>(&xk)[FT]) {
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < FT; i += 2) mma32(acc, Wf[i][o], Wf[i + 1][o], xk[i], xk[i + 1]);
      dst.pp[n >> 3][o >> 1][16 * g + (n & 7) + 8 * (o & 1)] = acc;
    }
  };
  // the saved slot's G, XH and row values of mini-batch s, and b_{s+1} = b_s - G_s^T e_s
  auto retire = [&](int s, const LinRowsPar<T, FT>& src, f4 e) {
    using Slot2 = LinSavedSlot<F>;
    const int sv = s * Slot2::BYTES;
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      f4 gv;
#pragma unroll
      for (int j = 0; j < 4; ++j) gv[j] = src.gx[0][o][4 * g + j][n];
      bstore_frag<float>(SV, 16 * l + 1024 * o, sv + Slot2::G, Frag<float>{gv});
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc += e[j] * gv[j];
      bn[o] -= sum_col4(acc);
    }
  };

  // prologue: P_0; b_{-1} = b_0; G_{-1} = 0, XK_{-1} = 0, M_{-1} = 0
  {
    LinRowsPar<T, FT>& pr = sh.par[1];
    Frag<T> Wf[FT][FT];
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) Wf[i][o] = to_frag<T>(W[i][o].v);
    put_p(pr, Wf, xk_cur);
    const u2v z2 = u2v{0u, 0u};
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      pr.gneg[o][l] = z2;
      pr.geta[o][l] = z2;
      sh.xkt[2][o][grow_put(o, n, g)] = z2;
      sh.xkt[0][o][grow_put(o, n, g)] = frag_bits(xk_cur[o]);
    }
    pr.mt[l] = z2;
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < FT; ++o) pr.b[16 * o + n] = bn[o];
    }
  }
  __syncthreads();  // prologue

  for (int s = 0; s < NC; ++s) {
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) asm volatile("" : "+v"(W[i][o].v));
    const ERow er = er_n;
    if (s + 2 < NC) load_xk(xk_pf, s + 2);
    if (s + 1 < NC) load_e(s + 1);
    LinRowsPar<T, FT>& cur = sh.par[s & 1];
    const LinRowsPar<T, FT>& prv = sh.par[(s + 1) & 1];

    // W_s = W_{s-1} - XK_{s-1}^T diag(e_{s-1}) G_{s-1}
    {
      Frag<T> geT[FT], xkT[FT];
#pragma unroll
      for (int o = 0; o < FT; ++o) geT[o] = lds_read_tr<T>(&prv.geta[o][grow_get(o, l)]);
#pragma unroll
      for (int i = 0; i < FT; ++i) xkT[i] = lds_read_tr<T>(&sh.xkt[(s + 2) % 3][i][grow_get(i, l)]);
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) mma16(W[i][o].v, xkT[i], geT[o]);
    }
    if (s > 0) retire(s - 1, prv, e_prev);  // b_s
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < FT; ++o) cur.b[16 * o + n] = bn[o];
    }
    if (p.W_ckpt != nullptr && (s % p.G) == 0) {
      const int kk = s / p.G;
      float* wc = p.W_ckpt + ((size_t)chain * p.NK + kk) * F * F;
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) store_tile(wc, F, 16 * i, 16 * o, W[i][o]);
      if (g == 0) {
#pragma unroll
        for (int o = 0; o < FT; ++o) p.b_ckpt[((size_t)chain * p.NK + kk) * F + 16 * o + n] = bn[o];
      }
    }
    {
      Frag<T> Wf[FT][FT];
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int o = 0; o < FT; ++o) {
          Wf[i][o] = to_frag<T>(W[i][o].v);
          cur.wf[o * FT + i][l] = Wf[i][o].v;
        }
      put_p(cur, Wf, xk_nxt);  // P_{s+1}
    }
    const f4 e = e_of(er);
    {
      // M_s^T frag: lane (g, n) = (XK_{s+1} XK_s^T + 1)[n][4g+j] e_s[4g+j]
      Tile cm[1][1];
      cm[0][0].v = f4{0.f, 0.f, 0.f, 0.f};
      Frag<T> a[1][FT], b[1][FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        a[0][c] = xk_cur[c];
        b[0][c] = xk_nxt[c];
      }
      gemm<1, 1, FT>(cm, a, b);
      cur.mt[l] = frag_bits(to_frag<T>((cm[0][0].v + 1.0f) * e));
    }
#pragma unroll
    for (int i = 0; i < FT; ++i) sh.xkt[(s + 1) % 3][i][grow_put(i, n, g)] = frag_bits(xk_nxt[i]);  // XK_{s+1}
#pragma unroll
    for (int c = 0; c < FT; ++c) {
      xk_cur[c] = xk_nxt[c];
      xk_nxt[c] = xk_pf[c];
    }
    e_prev = e;
    __syncthreads();  // mini-batch s handed over
  }

  // the last mini-batch's saved values; W_NC, b_NC
  const LinRowsPar<T, FT>& last = sh.par[(NC + 1) & 1];
  retire(NC - 1, last, e_prev);
  if (p.W_last != nullptr) {
    Frag<T> geT[FT], xkT[FT];
#pragma unroll
    for (int o = 0; o < FT; ++o) geT[o] = lds_read_tr<T>(&last.geta[o][grow_get(o, l)]);
#pragma unroll
    for (int i = 0; i < FT; ++i) xkT[i] = lds_read_tr<T>(&sh.xkt[(NC - 1) % 3][i][grow_get(i, l)]);
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) {
        mma16(W[i][o].v, xkT[i], geT[o]);
        store_tile(p.W_last + (size_t)chain * F * F, F, 16 * i, 16 * o, W[i][o]);
      }
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < FT; ++o) p.b_last[(size_t)chain * F + 16 * o + n] = bn[o];
    }
  }
}

template <typename T, int FT, bool LR, typename ET = T>
__global__ __launch_bounds__(256) void linear_fwd_rows_kernel(LinearFwdParams p) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  __shared__ LinRowsShared<T, FT> sh;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave == 0) {
    linear_rows_chain<T, FT, LR, ET, 0>(p, sh);
    return;
  }
  if (wave == 1) {
    linear_rows_chain<T, FT, LR, ET, 1>(p, sh);
    return;
  }
  if (wave == 2) {
    linear_rows_state<T, FT, LR, ET>(p, sh);
    return;
  }
  // ================================================================ wave O: the readout, one mini-batch behind
  const int chain = blockIdx.x;
  const int h = chain % p.H;
  const int NC = p.NC;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  const T* __restrict__ XQ = static_cast<const T*>(p.XQ) + (size_t)chain * NC * K * F;
  const T* __restrict__ XK = static_cast<const T*>(p.XK) + (size_t)chain * NC * K * F;
  const ET* __restrict__ ETA = LR ? nullptr : static_cast<const ET*>(p.eta) + (size_t)chain * NC * K * K;
  const float* __restrict__ LRP = LR ? static_cast<const float*>(p.eta) + (size_t)chain * NC * K : nullptr;
  using ERaw = std::conditional_t<LR, f4, Frag<ET>>;
  const int eta_rule = p.eta_rule;
  T* __restrict__ OUT = static_cast<T*>(p.out) + (size_t)chain * NC * K * F;
  using Slot = LinSavedSlot<F>;
  const rsrc_t SV = p.saved ? make_rsrc(static_cast<char*>(p.saved) + (size_t)chain * NC * Slot::BYTES,
                                        (unsigned)(NC * Slot::BYTES))
                            : make_rsrc(p.out, 0u);
  const float eps = p.eps;
  const float invF = 1.0f / F;
  f4 lnw_fm[FT], lnb_fm[FT];
#pragma unroll
  for (int o = 0; o < FT; ++o)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lnw_fm[o][j] = p.ln_w[h * F + 16 * o + 4 * g + j];
      lnb_fm[o][j] = p.ln_b[h * F + 16 * o + 4 * g + j];
    }
  Frag<T> nq[1][FT];
  ERaw n_etaT;
  auto load_step = [&](int s) {
    const T* q = XQ + (size_t)s * K * F;
#pragma unroll
    for (int c = 0; c < FT; ++c) nq[0][c] = load_frag(q, F, 16 * c);
    if constexpr (LR)
      n_etaT = *reinterpret_cast<const f4*>(LRP + (size_t)s * K + 4 * g);  // lane (g,*): lr[4g+j]
    else
      n_etaT = load_frag(ETA + (size_t)s * K * K, K, 0);  // lane (g,n): eta[n][4g+j]
  };
  load_step(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // prologue

  auto readout = [&](int s) {
    Frag<T> xq[1][FT], xk[1][FT];
#pragma unroll
    for (int c = 0; c < FT; ++c) {
      xq[0][c] = nq[0][c];
      xk[0][c] = bits_frag<T>(sh.xkt[s % 3][c][grow_put(c, n, g)]);  // XK_s (lane (g, n): row n)
    }
    const ERaw etaT_raw = n_etaT;
    if (s + 1 < NC) load_step(s + 1);
    const LinRowsPar<T, FT>& hs = sh.par[s & 1];
    const int sv = s * Slot::BYTES;
    // the saved slot's XH_s (token-major) and row values
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      f4 xv;
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[j] = hs.gx[1][o][4 * g + j][n];
      bstore_frag<float>(SV, 16 * l + 1024 * o, sv + Slot::XH, Frag<float>{xv});
    }
    bstore_frag<float>(SV, 16 * g, sv + Slot::RSTD, Frag<float>{*reinterpret_cast<const f4*>(&hs.rc[0][4 * g])});
    bstore_frag<float>(SV, 16 * g, sv + Slot::CC, Frag<float>{*reinterpret_cast<const f4*>(&hs.rc[1][4 * g])});

    // Zb^T = W^T XQ^T (feature-major) - G^T (eta o A + eta)^T + b
    Frag<T> Wf[FT][FT];
#pragma unroll
    for (int o = 0; o < FT; ++o)
#pragma unroll
      for (int i = 0; i < FT; ++i) Wf[o][i].v = hs.wf[o * FT + i][l];
    Tile zb[FT][1];
#pragma unroll
    for (int o = 0; o < FT; ++o) zb[o][0].v = *reinterpret_cast<const f4*>(&hs.b[16 * o + 4 * g]);
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
      for (int o = 0; o < FT; ++o) mma16(zb[o][0].v, lds_read_tr<T>(&hs.gneg[o][grow_get(o, l)]), mtf);
    }

    // ---- LN over features of each token (token n lives in lanes n, n+16, n+32, n+48)
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
  };
  for (int s = 0; s < NC; ++s) {
    if (s > 0) readout(s - 1);
    __syncthreads();  // mini-batch s handed over
  }
  readout(NC - 1);
}

template <typename T, int FT>
static hipError_t launch_rows(const LinearFwdParams& p, hipStream_t stream) {
  if (p.eta_rule == TTT_ETA_DENSE)
    hipLaunchKernelGGL((linear_fwd_rows_kernel<T, FT, false>), dim3(p.B * p.H), dim3(256), 0, stream, p);
  else if (p.eta_rule == TTT_ETA_DENSE_F32)
    hipLaunchKernelGGL((linear_fwd_rows_kernel<T, FT, false, float>), dim3(p.B * p.H), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((linear_fwd_rows_kernel<T, FT, true>), dim3(p.B * p.H), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_linear_fwd_rows(const LinearFwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_rows<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_rows<__bf16, 2>(p, stream);
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_rows<_Float16, 4>(p, stream);
    if (p.F == 32) return launch_rows<_Float16, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
