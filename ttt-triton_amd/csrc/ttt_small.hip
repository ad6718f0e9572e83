// Register-resident TTT inner loops for small heads on gfx950: mini-batches
// of K = 16..64 tokens (16 KT) with head dim F = 32 and, for the MLP, hidden
// width FF = 32 -- the reference's own model configuration (TTTMLP builds
// FF = F, ttt_layer.py:427-430; ModelConfig and main.py use K = 64 with model
// dim 128 over 4 heads, forecast.py:33-44, main.py:52-64).
//
// One wavefront per (batch, head) chain holds the whole fast-weight state (W1
// [F x FF] and W2 [FF x F] as fp32 MFMA accumulator tiles, 32 registers per
// lane at F = FF = 32) and all K tokens of a mini-batch, and walks the
// mini-batches in order (ops/ttt_mlp.py:9-67, ops/ttt_linear.py:8-54: dual
// form with the full K x K eta).  Every product is a set of 16 x 16 MFMA
// tiles (ttt_tile.h's gemm: Y = P Q^T from operand frags of P and Q); a
// token-by-feature matrix X is held either as C-layout tiles of X ("row
// layout": lane (g, n) has X[16i + 4g + j][16c + n]) or of X^T ("token
// layout": lane (g, n) has X[16i + n][16c + 4g + j], the layout of the
// activations' row-major loads and stores, and of the LayerNorms, which then
// reduce over four lanes).  A product contracting over features takes both
// operands in the token layout, one contracting over tokens both in the row
// layout; the few that need the other layout get it from an exact fp32
// transpose through the wave's own LDS (one 16-byte write and four 4-byte
// reads per tile, conflict-free with a padded stride).  With one wave per
// workgroup the LDS needs no barriers: a wave's LDS operations complete in
// issue order, and a compiler barrier keeps the program order.
//
// The forward stores the state entering every mini-batch in the caller's
// `saved` buffer (the general-shape layout, GenLayout); the backward visits
// the mini-batches in reverse, recomputes one mini-batch's forward values from
// its stored state and applies the hand-derived gradient of that mini-batch
// (through the update, the output LayerNorm, both dual-form attention
// products, GELU and its derivatives, and the LayerNorm fused with the L2
// loss), carrying the state gradient in registers.
#include "ttt_eta.h"
#include "ttt_kernels.h"

namespace ttt {
namespace {

struct SmallArgs {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b, *W1_init, *b1_init, *W2_init, *b2_init;
  void* out;
  float *last[4], *ckpt[4], *memo[4];  // W1, b1, W2, b2 of one chain's [n] state sets (may be null)
  void *dXQ, *dXK, *dXV, *deta;
  float *dW1, *db1, *dW2, *db2, *dln_w, *dln_b;
  float* saved;                     // per chain: GenLayout (the states entering each mini-batch first)
  float* hand;                      // MLP backward in two launches: one MlpBwdHand slot per (chain, mini-batch)
  size_t per_chain, states, state;  // floats
  int H, NC, G, M, NK, NS, eta_rule;
  float eps;
};

constexpr int kSmallMaxKT = 4;
constexpr int kStage = 16 * kSmallMaxKT * (16 * kSmallMaxKT + 4);  // transpose staging (floats)

// program order for the wave's LDS accesses (the hardware keeps issue order)
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

// C-layout tiles of X [16A x 16B] -> C-layout tiles of X^T, exact (fp32),
// through LDS: X^T row-major with a padded stride (writes of 16 bytes, reads
// of 4, each conflict-free over the lanes that share an access).
template <int A, int B> __device__ __forceinline__ void tr(const Tile (&x)[A][B], Tile (&y)[B][A], float* st) {
  constexpr int S = 16 * A + 4;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  lds_order();
#pragma unroll
  for (int i = 0; i < A; ++i)
#pragma unroll
    for (int j = 0; j < B; ++j) *reinterpret_cast<f4*>(st + (16 * j + n) * S + 16 * i + 4 * g) = x[i][j].v;
  lds_order();
#pragma unroll
  for (int j = 0; j < B; ++j)
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) y[j][i].v[jj] = st[(16 * j + 4 * g + jj) * S + 16 * i + n];
  lds_order();
}

// operand frags of X^T from C-layout tiles of X: f[b][a] = x[a][b] (cast)
template <typename T, int A, int B> __device__ __forceinline__ void frags_t(const Tile (&x)[A][B], Frag<T> (&f)[B][A]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) f[b][a] = to_frag<T>(x[a][b].v);
}
// same, every element times s (a per-register scale)
template <typename T, int A, int B>
__device__ __forceinline__ void frags_t_scaled(const Tile (&x)[A][B], const f4 (&s)[A], Frag<T> (&f)[B][A]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) f[b][a] = to_frag<T>(x[a][b].v * s[a]);
}
// token-layout fp32 tiles of X from its operand frags (the loaded activations)
template <typename T, int A, int B> __device__ __forceinline__ void tiles_of(const Frag<T> (&f)[A][B], Tile (&x)[B][A]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) x[b][a].v = frag_to_f4(f[a][b]);
}
template <int A, int B> __device__ __forceinline__ void zero(Tile (&x)[A][B]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) x[a][b].v = f4{0.f, 0.f, 0.f, 0.f};
}
// fp32 tiles parked in LDS in lane order (one 16-byte access per lane and tile)
template <int A, int B> __device__ __forceinline__ void park(float* p, const Tile (&x)[A][B]) {
  lds_order();
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) *reinterpret_cast<f4*>(p + ((a * B + b) * 64 + lane_id()) * 4) = x[a][b].v;
  lds_order();
}
template <int A, int B> __device__ __forceinline__ void unpark(const float* p, Tile (&x)[A][B]) {
  lds_order();
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) x[a][b].v = *reinterpret_cast<const f4*>(p + ((a * B + b) * 64 + lane_id()) * 4);
  lds_order();
}

__device__ __forceinline__ float hsum(f4 v) { return (v[0] + v[1]) + (v[2] + v[3]); }
__device__ __forceinline__ f4 sum_row16_4(f4 v) {
  return f4{sum_row16(v[0]), sum_row16(v[1]), sum_row16(v[2]), sum_row16(v[3])};
}

// The mini-batch's activations, and its eta on demand (dense or from lr).
template <typename T, int KT, int FT> struct SmallInputs {
  Frag<T> q[KT][FT], k[KT][FT], v[KT][FT];  // XQ, XK, XV frags (free = token): token layout
  f4 e4[KT];                                 // last row eta[K-1][16i + 4g + jj] (row layout scale)
  float eT[KT];                              // eta[K-1][16i + n] (token layout scale)
  const T* E;                                // dense: this mini-batch's [K][K] block
  const float* EF;                           // dense fp32 eta: the same block
  const float* lr;                           // lr form: this mini-batch's [K] rates
  int rule;

  __device__ __forceinline__ void load(const SmallArgs& a, size_t row0) {
    constexpr int K = 16 * KT, F = 16 * FT;
    const int l = lane_id(), g = l >> 4, n = l & 15;
    const T* XQ = static_cast<const T*>(a.XQ) + row0 * F;
    const T* XK = static_cast<const T*>(a.XK) + row0 * F;
    const T* XV = static_cast<const T*>(a.XV) + row0 * F;
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int j = 0; j < FT; ++j) {
        q[i][j] = load_frag(XQ + 16 * i * F, F, 16 * j);
        k[i][j] = load_frag(XK + 16 * i * F, F, 16 * j);
        v[i][j] = load_frag(XV + 16 * i * F, F, 16 * j);
      }
    rule = a.eta_rule;
    if (rule == TTT_ETA_DENSE) {
      E = static_cast<const T*>(a.eta) + row0 * K;
      EF = nullptr;
      lr = nullptr;
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        e4[i] = load4(E + (size_t)(K - 1) * K + 16 * i + 4 * g);
        eT[i] = (float)E[(size_t)(K - 1) * K + 16 * i + n];
      }
    } else if (rule == TTT_ETA_DENSE_F32) {
      E = nullptr;
      EF = static_cast<const float*>(a.eta) + row0 * K;
      lr = nullptr;
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        e4[i] = load4(EF + (size_t)(K - 1) * K + 16 * i + 4 * g);
        eT[i] = EF[(size_t)(K - 1) * K + 16 * i + n];
      }
    } else {
      E = nullptr;
      EF = nullptr;
      lr = static_cast<const float*>(a.eta) + row0;
      const float invK = 1.0f / (float)K;
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        e4[i] = *reinterpret_cast<const f4*>(lr + 16 * i + 4 * g) * invK;  // row K-1: 1/K under both rules
        eT[i] = lr[16 * i + n] * invK;
      }
    }
  }
  // eta[16i + n][16j + 4g + jj] (lane (g, n)) as et[i][j]
  __device__ __forceinline__ void eta(f4 (&et)[KT][KT]) const {
    constexpr int K = 16 * KT;
    const int l = lane_id(), g = l >> 4, n = l & 15;
    if (rule == TTT_ETA_DENSE) {
#pragma unroll
      for (int i = 0; i < KT; ++i)
#pragma unroll
        for (int j = 0; j < KT; ++j) et[i][j] = frag_to_f4(load_frag(E + 16 * i * K, K, 16 * j));
    } else if (rule == TTT_ETA_DENSE_F32) {
#pragma unroll
      for (int i = 0; i < KT; ++i)
#pragma unroll
        for (int j = 0; j < KT; ++j) et[i][j] = frag_to_f4(load_frag(EF + 16 * i * K, K, 16 * j));
    } else {
      const bool layer = rule == TTT_ETA_LAYER;
      const float invK = 1.0f / (float)K;
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        const float c = 1.0f / (float)(16 * i + n + 1);  // causal coefficient of row 16i + n
#pragma unroll
        for (int j = 0; j < KT; ++j) {
          const f4 lr4 = *reinterpret_cast<const f4*>(lr + 16 * j + 4 * g);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            et[i][j][jj] = layer ? lr4[jj] * invK : (16 * j + 4 * g + jj <= 16 * i + n ? lr4[jj] * c : 0.0f);
        }
      }
    }
  }
};

// LayerNorm statistics of one token-layout row set (lane (g, n): token n,
// features 16c + 4g + jj): mean and 1/sigma over F features
template <int FT> __device__ __forceinline__ void ln_stats(const f4 (&z)[FT], float eps, float& mu, float& rs) {
  constexpr float invF = 1.0f / (16 * FT);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < FT; ++c) s += hsum(z[c]);
  mu = sum_col4(s) * invF;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    const f4 d = z[c] - mu;
    q += hsum(d * d);
  }
  rs = rsqrt_f(sum_col4(q) * invF + eps);
}

// ln_fused_l2_bwd (ops/ttt_utils.py:21-48) on token-layout rows: G from
// Z and the target; xh = normalised Z
template <int FT>
__device__ __forceinline__ void ln_l2_fwd(const f4 (&z)[FT], const f4 (&tgt)[FT], const f4 (&lw)[FT],
                                          const f4 (&lb)[FT], float eps, f4 (&xh)[FT], f4 (&G)[FT], float& rs) {
  constexpr float invF = 1.0f / (16 * FT);
  float mu;
  ln_stats<FT>(z, eps, mu, rs);
  f4 gx[FT];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    xh[c] = (z[c] - mu) * rs;
    gx[c] = (lw[c] * xh[c] + lb[c] - tgt[c]) * lw[c];
    s1 += hsum(gx[c]);
    s2 += hsum(gx[c] * xh[c]);
  }
  s1 = sum_col4(s1) * invF;
  s2 = sum_col4(s2) * invF;
#pragma unroll
  for (int c = 0; c < FT; ++c) G[c] = (gx[c] - s1 - xh[c] * s2) * rs;
}

// The backward of ln_fused_l2_bwd on token-layout rows (the derivation of
// ttt_generic.hip): from dG (qv) and the forward's xh, G, 1/sigma and
// target, dZ; dXV (= dt) and the LayerNorm parameters' terms
template <int FT>
__device__ __forceinline__ void ln_l2_bwd(const f4 (&xh)[FT], const f4 (&qv)[FT], const f4 (&G)[FT],
                                          const f4 (&tgt)[FT], const f4 (&lw)[FT], const f4 (&lb)[FT], float rs,
                                          f4 (&dz)[FT], f4 (&dt)[FT], f4 (&dlw)[FT], f4 (&dlb)[FT]) {
  constexpr int F = 16 * FT;
  constexpr float invF = 1.0f / F;
  f4 rr[FT], gg[FT];
  float S2 = 0.f, Q1 = 0.f, Q2 = 0.f, QG = 0.f;
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    rr[c] = lw[c] * xh[c] + lb[c] - tgt[c];
    gg[c] = lw[c] * rr[c];
    S2 += hsum(gg[c] * xh[c]);
    Q1 += hsum(qv[c]);
    Q2 += hsum(qv[c] * xh[c]);
    QG += hsum(qv[c] * G[c]);
  }
  S2 = sum_col4(S2);
  Q1 = sum_col4(Q1);
  Q2 = sum_col4(Q2);
  QG = sum_col4(QG);
  const float inv = rs * invF;
  const float dsig = -QG * rs;
  float m1 = 0.f, m2 = 0.f;
  f4 dxh[FT];
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    const f4 dg = ((float)F * qv[c] - Q1 - xh[c] * Q2) * inv;
    dxh[c] = (-qv[c] * S2 - gg[c] * Q2) * inv + dg * lw[c] * lw[c];
    dt[c] = -dg * lw[c];
    dlw[c] += dg * (rr[c] + lw[c] * xh[c]);
    dlb[c] += dg * lw[c];
    m1 += hsum(dxh[c]);
    m2 += hsum(dxh[c] * xh[c]);
  }
  m1 = sum_col4(m1) * invF;
  m2 = sum_col4(m2) * invF;
#pragma unroll
  for (int c = 0; c < FT; ++c) dz[c] = (dxh[c] - m1 - xh[c] * m2) * rs + dsig * xh[c] * invF;
}

// The output LayerNorm's backward on token-layout rows: out = XQ + lw xhb + lb
template <int FT>
__device__ __forceinline__ void ln_out_bwd(const f4 (&dout)[FT], const f4 (&xhb)[FT], const f4 (&lw)[FT], float rs,
                                           f4 (&dz)[FT], f4 (&dlw)[FT], f4 (&dlb)[FT]) {
  constexpr float invF = 1.0f / (16 * FT);
  f4 dh[FT];
  float m1 = 0.f, m2 = 0.f;
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    dh[c] = dout[c] * lw[c];
    m1 += hsum(dh[c]);
    m2 += hsum(dh[c] * xhb[c]);
    dlw[c] += dout[c] * xhb[c];
    dlb[c] += dout[c];
  }
  m1 = sum_col4(m1) * invF;
  m2 = sum_col4(m2) * invF;
#pragma unroll
  for (int c = 0; c < FT; ++c) dz[c] = (dh[c] - m1 - xhb[c] * m2) * rs;
}

// the eta gradient's last row also carries de (the update's eta); stored
// dense, or as dlr = sum over rows of deta * coef under the rule
template <typename T, int KT>
__device__ __forceinline__ void store_deta(const SmallArgs& a, size_t row0, const Tile (&detaT)[KT][KT],
                                           const float* sde) {
  constexpr int K = 16 * KT;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  f4 de_row[KT];  // de[16j + 4g + jj]
#pragma unroll
  for (int j = 0; j < KT; ++j) de_row[j] = *reinterpret_cast<const f4*>(sde + 16 * j + 4 * g);
  if (a.eta_rule == TTT_ETA_DENSE || a.eta_rule == TTT_ETA_DENSE_F32) {
    T* DE = static_cast<T*>(a.deta) + row0 * K;
    float* DEF = static_cast<float*>(a.deta) + row0 * K;
    const bool f32 = a.eta_rule == TTT_ETA_DENSE_F32;
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        f4 v = detaT[j][i].v;
        if (i == KT - 1 && n == 15) v += de_row[j];
        if (f32)
          store_f4(DEF + 16 * i * K, K, 16 * j, v);
        else
          store_f4(DE + 16 * i * K, K, 16 * j, v);
      }
  } else {
    float* DL = static_cast<float*>(a.deta) + row0;
    const bool layer = a.eta_rule == TTT_ETA_LAYER;
    const float invK = 1.0f / (float)K;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        const float c = 1.0f / (float)(16 * i + n + 1);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          acc[jj] += detaT[j][i].v[jj] * (layer ? invK : (16 * j + 4 * g + jj <= 16 * i + n ? c : 0.0f));
      }
      acc = sum_row16_4(acc) + de_row[j] * invK;
      if (n == 0) store4(DL + 16 * j + 4 * g, acc);
    }
  }
}

// deta's last row (or dlr) gains the update path's term de of column j: the
// second launch of the two-launch MLP backward adds it to what the first
// stored (dense: eta[K-1][j]; lr rules: dlr[j] with the last row's 1/K)
template <typename T>
__device__ __forceinline__ void add_deta_last_row(const SmallArgs& a, size_t row0, int K, int j, float de) {
  if (a.eta_rule == TTT_ETA_DENSE) {
    T* p = static_cast<T*>(a.deta) + (row0 + K - 1) * K + j;
    float v = (float)*p + de;
    asm("" : "+v"(v));  // (a plain conversion, as f16x4_of keeps them)
    *p = (T)v;
  } else if (a.eta_rule == TTT_ETA_DENSE_F32) {
    static_cast<float*>(a.deta)[(row0 + K - 1) * K + j] += de;
  } else {
    static_cast<float*>(a.deta)[row0 + j] += de * (1.0f / (float)K);
  }
}

// token-layout [FT][KT] tiles -> rows of a [K x F] activation block
template <typename T, int KT, int FT>
__device__ __forceinline__ void store_rows(void* base, size_t row0, const Tile (&xT)[FT][KT]) {
  constexpr int F = 16 * FT;
  T* X = static_cast<T*>(base) + row0 * F;
#pragma unroll
  for (int i = 0; i < KT; ++i)
#pragma unroll
    for (int c = 0; c < FT; ++c) store_f4(X + 16 * i * F, F, 16 * c, xT[c][i].v);
}

// ---------------------------------------------------------------- TTT-MLP
//
// Per mini-batch (Z1 = XK W1 + b1 etc., ops/ttt_mlp.py:28-56), with layouts:
//   Z1, X2 = gelu(Z1), gelu'(Z1), P1 = G2 W2^T, G1 = P1 gelu'(Z1)    row
//   X2 (also), Z2, G2 (also row), Z1b, X2b, Z2b, output               token
//   A1 = XQ XK^T, A2 = X2b X2^T, eta, C = eta (A + 1): tiles [t'][t] of the
//   token layout of [t x t'] (lane (g, n): row 16i + n, column 16j + 4g + jj)
// The values later phases read are parked in the wave's LDS (lane order),
// so that only the phase at hand holds registers.
template <int KT, int FT, int HT, bool FULL> struct MlpPark {
  static constexpr int R = KT * HT * 256;   // a [KT][HT] tile set, floats
  static constexpr int TF = FT * KT * 256;  // [FT][KT]
  static constexpr int KK = KT * KT * 256;  // [KT][KT]
  static constexpr int X2 = 0;              // X2 (row)
  static constexpr int G1 = X2 + R;         // G1 (row)
  static constexpr int G2T = G1 + R;        // G2 (token)
  // backward only: more forward values, then the gradients that several
  // phases add to
  static constexpr int D1 = G2T + TF;                 // gelu'(Z1) (row)
  static constexpr int PDD = D1 + (FULL ? R : 0);     // P1 gelu''(Z1) (row)
  static constexpr int XH2T = PDD + (FULL ? R : 0);   // normalised Z2 (token)
  static constexpr int X2BT = XH2T + (FULL ? TF : 0); // X2b (token)
  static constexpr int DB1T = X2BT + (FULL ? R : 0);  // gelu'(Z1b) (token)
  static constexpr int XHBT = DB1T + (FULL ? R : 0);  // normalised Z2b (token)
  static constexpr int DX2 = XHBT + (FULL ? TF : 0);  // dX2 (row)
  static constexpr int DG2T = DX2 + (FULL ? R : 0);   // dG2 (token)
  static constexpr int DXKT = DG2T + (FULL ? TF : 0); // dXK (token)
  static constexpr int DETA = DXKT + (FULL ? TF : 0); // deta, tiles [t'][t]
  static constexpr int FLOATS = DETA + (FULL ? KK : 0);
};
// The readout-path launch of the two-launch backward parks only what its
// phases read back (its update-path values are not formed, the normalised
// Z2b rows stay in registers and its dG2, dX2 and dXK terms go straight to
// the handoff): 56 KB at K = 64, so that two workgroups share a CU.
template <int KT, int FT, int HT> struct MlpParkRO {
  static constexpr int R = KT * HT * 256, TF = FT * KT * 256, KK = KT * KT * 256;
  static constexpr int X2 = 0, G1 = X2 + R, G2T = G1 + R, X2BT = G2T + TF, DB1T = X2BT + R, DETA = DB1T + R;
  static constexpr int FLOATS = DETA + KK;
};

// The MLP backward's handoff slot per (chain, mini-batch), floats, every set
// in lane order (one 16-byte vector per lane and tile): the readout path's
// terms of dG1 (row), dG2 (token), dX2 (row), dXK (token), of the state
// gradients dW1, dW2 (C layout), of db1 (token sums), db2 (per lane) and of
// the output LayerNorm parameters' gradients (per lane).
template <int KT, int FT, int HT> struct MlpBwdHand {
  static constexpr int R = KT * HT * 256, TF = FT * KT * 256, WW = FT * HT * 256;
  static constexpr int DG1 = 0, DG2T = DG1 + R, DX2 = DG2T + TF, DXKT = DX2 + R, DW1 = DXKT + TF, DW2 = DW1 + WW;
  static constexpr int DB1T = DW2 + WW, DB2C = DB1T + HT * 256, DLNW = DB2C + FT * 256, DLNB = DLNW + FT * 256;
  static constexpr int FLOATS = DLNB + FT * 256;
};
template <int A, int B> __device__ __forceinline__ void hand_store(float* p, const Tile (&x)[A][B]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) *reinterpret_cast<f4*>(p + ((a * B + b) * 64 + lane_id()) * 4) = x[a][b].v;
}
template <int A, int B> __device__ __forceinline__ void hand_add(const float* p, Tile (&x)[A][B]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) x[a][b].v += *reinterpret_cast<const f4*>(p + ((a * B + b) * 64 + lane_id()) * 4);
}
template <int N> __device__ __forceinline__ void hand_store4(float* p, const f4 (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) *reinterpret_cast<f4*>(p + (i * 64 + lane_id()) * 4) = x[i];
}
template <int N> __device__ __forceinline__ void hand_load4(const float* p, f4 (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] = *reinterpret_cast<const f4*>(p + (i * 64 + lane_id()) * 4);
}

// One mini-batch's forward values from the state entering it; parks what
// the caller's later phases need, returns the output rows (token layout) and
// the two LayerNorms' 1/sigma per token tile.  Without RO it stops after G1
// (the inner loss's values only: no readout, rsb and outT left unset).
// UPV parks the update path's values (gelu'(Z1), P1 gelu''(Z1), the
// normalised Z2); XHB_OUT returns the normalised Z2b rows in outT instead of
// the output rows and parks none.  P is the park layout.
template <typename T, int KT, int FT, int HT, bool FULL, bool RO = true, typename P = MlpPark<KT, FT, HT, FULL>,
          bool UPV = FULL, bool XHB_OUT = false>
__device__ __forceinline__ void mlp_step(const SmallInputs<T, KT, FT>& in, const Tile (&W1)[FT][HT],
                                         const Tile (&W2)[HT][FT], const float (&b1n)[HT], const f4 (&b1T)[HT],
                                         const f4 (&b2T)[FT], const f4 (&lw)[FT], const f4 (&lb)[FT], float eps,
                                         float* st, float* pk, float (&rs2)[KT], float (&rsb)[KT],
                                         Tile (&outT)[FT][KT]) {
  Frag<T> fW1t[HT][FT], fW2t[FT][HT], fW2[HT][FT];
  frags_t<T>(W1, fW1t);
  frags_t<T>(W2, fW2t);
  {
    Tile w2T[FT][HT];
    tr(W2, w2T, st);
    frags_t<T>(w2T, fW2);
  }
  // Z1 = XK W1 + b1 (row layout), gelu and its derivatives
  Frag<T> fX2[KT][HT];  // X2 frags (free = token)
  Tile d1[KT][HT];
  {
    Tile z1[KT][HT], x2[KT][HT];
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) z1[i][o].v = f4{b1n[o], b1n[o], b1n[o], b1n[o]};
    gemm<KT, HT, FT>(z1, in.k, fW1t);
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float y, dy, ddy;
          if constexpr (UPV) {
            gelu_all(z1[i][o].v[jj], y, dy, ddy);
            z1[i][o].v[jj] = ddy;  // (z1 now holds gelu''(Z1))
          } else {
            gelu_fwd_bwd(z1[i][o].v[jj], y, dy);
          }
          x2[i][o].v[jj] = y;
          d1[i][o].v[jj] = dy;
        }
    park(pk + P::X2, x2);
    Tile x2T[HT][KT];
    tr(x2, x2T, st);
    frags_t<T>(x2T, fX2);
    if constexpr (UPV) {
      park(pk + P::D1, d1);
      park(pk + P::PDD, z1);  // gelu''(Z1) for now; times P1 below
    }
  }
  // Z2 (token layout) and the inner loss's gradient G2
  Frag<T> fG2[KT][FT];
  {
    Tile z2T[FT][KT];
#pragma unroll
    for (int c = 0; c < FT; ++c)
#pragma unroll
      for (int i = 0; i < KT; ++i) z2T[c][i].v = b2T[c];
    gemm<FT, KT, HT>(z2T, fW2t, fX2);
    Tile g2T[FT][KT], xh2T[FT][KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) {
      f4 z[FT], tg[FT], xh[FT], G[FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        z[c] = z2T[c][i].v;
        tg[c] = frag_to_f4(in.v[i][c]) - frag_to_f4(in.k[i][c]);
      }
      ln_l2_fwd<FT>(z, tg, lw, lb, eps, xh, G, rs2[i]);
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        g2T[c][i].v = G[c];
        xh2T[c][i].v = xh[c];
      }
    }
    frags_t<T>(g2T, fG2);
    park(pk + P::G2T, g2T);
    if constexpr (UPV) park(pk + P::XH2T, xh2T);
  }
  // P1 = G2 W2^T, G1 = P1 gelu'(Z1) (row layout)
  Frag<T> fG1t[HT][KT];
  {
    Tile p1[KT][HT];
    zero(p1);
    gemm<KT, HT, FT>(p1, fG2, fW2);
    if constexpr (UPV) {
      Tile pdd[KT][HT];
      unpark(pk + P::PDD, pdd);
#pragma unroll
      for (int i = 0; i < KT; ++i)
#pragma unroll
        for (int o = 0; o < HT; ++o) pdd[i][o].v *= p1[i][o].v;
      park(pk + P::PDD, pdd);
    }
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) p1[i][o].v *= d1[i][o].v;  // G1
    park(pk + P::G1, p1);
    frags_t<T>(p1, fG1t);
  }
  if constexpr (!RO) return;
  // A1 = XQ XK^T; Z1b = XQ W1 + b1 - (eta (A1 + 1)) G1 (token layout)
  f4 eta[KT][KT];
  in.eta(eta);
  Frag<T> fX2b[KT][HT];
  {
    Tile a1T[KT][KT];
    zero(a1T);
    gemm<KT, KT, FT>(a1T, in.k, in.q);
#pragma unroll
    for (int j = 0; j < KT; ++j)
#pragma unroll
      for (int i = 0; i < KT; ++i) a1T[j][i].v += 1.0f;
    Frag<T> fnC1[KT][KT];
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int j = 0; j < KT; ++j) fnC1[i][j] = to_frag<T>(-(eta[i][j] * a1T[j][i].v));
    Tile z1bT[HT][KT];
#pragma unroll
    for (int o = 0; o < HT; ++o)
#pragma unroll
      for (int i = 0; i < KT; ++i) z1bT[o][i].v = b1T[o];
    gemm<HT, KT, FT>(z1bT, fW1t, in.q);
    gemm<HT, KT, KT>(z1bT, fG1t, fnC1);
    Tile x2bT[HT][KT];
#pragma unroll
    for (int o = 0; o < HT; ++o)
#pragma unroll
      for (int i = 0; i < KT; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float y, dy;
          if constexpr (FULL) {
            gelu_fwd_bwd(z1bT[o][i].v[jj], y, dy);
            z1bT[o][i].v[jj] = dy;  // (z1bT now holds gelu'(Z1b))
          } else {
            y = gelu_tanh(z1bT[o][i].v[jj]);
          }
          x2bT[o][i].v[jj] = y;
        }
    frags_t<T>(x2bT, fX2b);
    if constexpr (FULL) {
      park(pk + P::X2BT, x2bT);
      park(pk + P::DB1T, z1bT);
    }
  }
  // A2 = X2b X2^T; Z2b = X2b W2 + b2 - (eta (A2 + 1)) G2 (token layout)
  {
    Tile a2T[KT][KT];
    zero(a2T);
    gemm<KT, KT, HT>(a2T, fX2, fX2b);
#pragma unroll
    for (int j = 0; j < KT; ++j)
#pragma unroll
      for (int i = 0; i < KT; ++i) a2T[j][i].v += 1.0f;
    Frag<T> fnC2[KT][KT], fG2t[FT][KT];
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int j = 0; j < KT; ++j) fnC2[i][j] = to_frag<T>(-(eta[i][j] * a2T[j][i].v));
    {
      Tile g2T[FT][KT], g2R[KT][FT];
      unpark(pk + P::G2T, g2T);
      tr(g2T, g2R, st);
      frags_t<T>(g2R, fG2t);
    }
    Tile z2bT[FT][KT];
#pragma unroll
    for (int c = 0; c < FT; ++c)
#pragma unroll
      for (int i = 0; i < KT; ++i) z2bT[c][i].v = b2T[c];
    gemm<FT, KT, HT>(z2bT, fW2t, fX2b);
    gemm<FT, KT, KT>(z2bT, fG2t, fnC2);
    // output LayerNorm and residual (ln_fwd, ops/ttt_utils.py:4-18)
    Tile xhbT[FT][KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) {
      f4 z[FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) z[c] = z2bT[c][i].v;
      float mu;
      ln_stats<FT>(z, eps, mu, rsb[i]);
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        xhbT[c][i].v = (z[c] - mu) * rsb[i];
        if constexpr (XHB_OUT)
          outT[c][i].v = xhbT[c][i].v;
        else
          outT[c][i].v = frag_to_f4(in.q[i][c]) + lw[c] * xhbT[c][i].v + lb[c];
      }
    }
    if constexpr (FULL && !XHB_OUT) park(pk + P::XHBT, xhbT);
  }
}

// state <-> global: W1 [F][FF], b1 [FF], W2 [FF][F], b2 [F] row-major (one chain)
template <int FT, int HT>
__device__ __forceinline__ void load_mlp_state(const float* W1, const float* b1, const float* W2, const float* b2,
                                               Tile (&cW1)[FT][HT], Tile (&cW2)[HT][FT], float* sb1, f4 (&b2T)[FT]) {
  constexpr int F = 16 * FT, FF = 16 * HT;
  const int l = lane_id(), g = l >> 4;
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < HT; ++o) cW1[i][o] = load_tile(W1, FF, 16 * i, 16 * o);
#pragma unroll
  for (int o = 0; o < HT; ++o)
#pragma unroll
    for (int c = 0; c < FT; ++c) cW2[o][c] = load_tile(W2, F, 16 * o, 16 * c);
  lds_order();
  if (l < FF) sb1[l] = b1[l];
  lds_order();
#pragma unroll
  for (int c = 0; c < FT; ++c) b2T[c] = load4(b2 + 16 * c + 4 * g);
}
template <int FT, int HT>
__device__ __forceinline__ void store_mlp_state(float* W1, float* b1, float* W2, float* b2, const Tile (&cW1)[FT][HT],
                                                const Tile (&cW2)[HT][FT], const float* sb1, const f4 (&b2T)[FT]) {
  constexpr int F = 16 * FT, FF = 16 * HT;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  if (W1 != nullptr) {
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) store_tile(W1, FF, 16 * i, 16 * o, cW1[i][o]);
  }
  if (b1 != nullptr && l < FF) b1[l] = sb1[l];
  if (W2 != nullptr) {
#pragma unroll
    for (int o = 0; o < HT; ++o)
#pragma unroll
      for (int c = 0; c < FT; ++c) store_tile(W2, F, 16 * o, 16 * c, cW2[o][c]);
  }
  if (b2 != nullptr && n == 0) {
#pragma unroll
    for (int c = 0; c < FT; ++c) store4(b2 + 16 * c + 4 * g, b2T[c]);
  }
}

template <int FT> __device__ __forceinline__ void load_ln(const SmallArgs& a, int h, f4 (&lw)[FT], f4 (&lb)[FT]) {
  constexpr int F = 16 * FT;
  const int g = lane_id() >> 4;
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    lw[c] = load4(a.ln_w + h * F + 16 * c + 4 * g);
    lb[c] = load4(a.ln_b + h * F + 16 * c + 4 * g);
  }
}

template <typename T, int KT, int FT, int HT>
__global__ __launch_bounds__(64) void small_mlp_fwd_kernel(SmallArgs a) {
  constexpr int K = 16 * KT, F = 16 * FT, FF = 16 * HT;
  using P = MlpPark<KT, FT, HT, false>;
  __shared__ __align__(16) float st[kStage];
  __shared__ __align__(16) float pk[P::FLOATS];
  __shared__ __align__(16) float sb1[FF];
  const size_t chain = blockIdx.x;
  const int h = (int)(chain % a.H), NC = a.NC;
  const int l = lane_id(), g = l >> 4, n = l & 15;

  Tile cW1[FT][HT], cW2[HT][FT];
  f4 b2T[FT];
  load_mlp_state<FT, HT>(a.W1_init + chain * F * FF, a.b1_init + chain * FF, a.W2_init + chain * FF * F,
                         a.b2_init + chain * F, cW1, cW2, sb1, b2T);
  f4 lw[FT], lb[FT];
  load_ln<FT>(a, h, lw, lb);
  float* states = a.saved + chain * a.per_chain + a.states;
  auto state_ptrs = [&](float* const (&d)[4], size_t k, float*& w1, float*& b1, float*& w2, float*& b2) {
    w1 = d[0] ? d[0] + k * F * FF : nullptr;
    b1 = d[1] ? d[1] + k * FF : nullptr;
    w2 = d[2] ? d[2] + k * FF * F : nullptr;
    b2 = d[3] ? d[3] + k * F : nullptr;
  };

  for (int s = 0; s < NC; ++s) {
    {
      float* S = states + (size_t)s * a.state;  // the state entering mini-batch s (the backward's)
      store_mlp_state<FT, HT>(S, S + F * FF, S + F * FF + FF, S + F * FF + FF + FF * F, cW1, cW2, sb1, b2T);
    }
    if (a.ckpt[0] != nullptr && s % a.G == 0) {
      float *w1, *b1, *w2, *b2;
      state_ptrs(a.ckpt, chain * a.NK + s / a.G, w1, b1, w2, b2);
      store_mlp_state<FT, HT>(w1, b1, w2, b2, cW1, cW2, sb1, b2T);
    }
    const size_t row0 = ((size_t)chain * NC + s) * K;
    SmallInputs<T, KT, FT> in;
    in.load(a, row0);
    float b1n[HT];
    f4 b1T[HT];
    lds_order();
#pragma unroll
    for (int o = 0; o < HT; ++o) {
      b1n[o] = sb1[16 * o + n];
      b1T[o] = *reinterpret_cast<const f4*>(sb1 + 16 * o + 4 * g);
    }
    {
      float rs2[KT], rsb[KT];
      Tile outT[FT][KT];
      mlp_step<T, KT, FT, HT, false>(in, cW1, cW2, b1n, b1T, b2T, lw, lb, a.eps, st, pk, rs2, rsb, outT);
      store_rows<T, KT, FT>(a.out, row0, outT);
    }
    // state update with the last eta row e (ops/ttt_mlp.py:48-52):
    // W1 -= XK^T diag(e) G1, W2 -= X2^T diag(e) G2, b1 -= G1^T e, b2 -= G2^T e
    {
      f4 ne[KT];
#pragma unroll
      for (int i = 0; i < KT; ++i) ne[i] = -in.e4[i];
      {
        Tile xkT[FT][KT], xkR[KT][FT], g1[KT][HT];
        tiles_of<T>(in.k, xkT);
        tr(xkT, xkR, st);
        Frag<T> fXKt[FT][KT], fnG1e[HT][KT];
        frags_t<T>(xkR, fXKt);
        unpark(pk + P::G1, g1);
        frags_t_scaled<T>(g1, ne, fnG1e);
        gemm<FT, HT, KT>(cW1, fXKt, fnG1e);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < KT; ++i) d += hsum(in.e4[i] * g1[i][o].v);
          d = sum_col4(d);
          if (g == 0) sb1[16 * o + n] = b1n[o] - d;
        }
      }
      {
        Tile x2[KT][HT], g2T[FT][KT], g2R[KT][FT];
        unpark(pk + P::X2, x2);
        unpark(pk + P::G2T, g2T);
        tr(g2T, g2R, st);
        Frag<T> fX2t[HT][KT], fnG2e[FT][KT];
        frags_t<T>(x2, fX2t);
        frags_t_scaled<T>(g2R, ne, fnG2e);
        gemm<HT, FT, KT>(cW2, fX2t, fnG2e);
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          f4 d = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < KT; ++i) d += in.eT[i] * g2T[c][i].v;
          b2T[c] -= sum_row16_4(d);
        }
      }
      lds_order();
    }
    if (a.memo[0] != nullptr && s % a.M == 0) {
      float *w1, *b1, *w2, *b2;
      state_ptrs(a.memo, chain * a.NS + s / a.M, w1, b1, w2, b2);
      store_mlp_state<FT, HT>(w1, b1, w2, b2, cW1, cW2, sb1, b2T);
    }
  }
  if (a.last[0] != nullptr) {
    float *w1, *b1, *w2, *b2;
    state_ptrs(a.last, chain, w1, b1, w2, b2);
    store_mlp_state<FT, HT>(w1, b1, w2, b2, cW1, cW2, sb1, b2T);
  }
}

// The gradient of one mini-batch (the derivation the general-shape kernel
// applies, ttt_generic.hip), with the state gradient dW1, dW2 (C-layout
// tiles), db1 (LDS, feature order), db2 (token-layout form) carried from the
// mini-batch after, in phases that each read their forward values back from
// the park, where the gradients several phases add to also wait; see the
// layout notes above MlpPark.
//
// MODE 0 runs every phase in one reverse sweep per chain.  The phases of the
// readout path, (2)-(4), do not depend on the state gradient carried from
// the later mini-batches, so with a handoff buffer the backward runs as two
// launches: MODE 1, one wave per (chain, mini-batch) at once, runs (2)-(4),
// stores dXQ and deta without the last row's update term, and leaves its
// contributions to dG1, dG2, dX2, dXK, the state gradients and the LayerNorm
// parameters' gradients in the handoff slot; MODE 2, the reverse sweep per
// chain, runs (1) and (5)-(7), adds each mini-batch's slot after (1) and the
// update term to deta's last row.
template <typename T, int KT, int FT, int HT, int MODE = 0>
__global__ __launch_bounds__(64) void small_mlp_bwd_kernel(SmallArgs a) {
  constexpr int K = 16 * KT, F = 16 * FT, FF = 16 * HT;
  constexpr bool RO = MODE != 2;  // the readout path's phases (2)-(4)
  constexpr bool UP = MODE != 1;  // the update path's phases (1), (5)-(7) and the carried state gradient
  using P = std::conditional_t<MODE == 1, MlpParkRO<KT, FT, HT>, MlpPark<KT, FT, HT, true>>;
  using HS = MlpBwdHand<KT, FT, HT>;
  __shared__ __align__(16) float st[kStage];
  __shared__ __align__(16) float pk[P::FLOATS];
  __shared__ __align__(16) float sb1[FF];
  __shared__ __align__(16) float sdb1[FF];
  __shared__ __align__(16) float sde[K];
  const size_t chain = MODE == 1 ? blockIdx.x / a.NC : blockIdx.x;
  const int h = (int)(chain % a.H), NC = a.NC;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  // MODE 1: this workgroup's one mini-batch
  const int s_hi = MODE == 1 ? (int)(blockIdx.x % a.NC) : NC - 1, s_lo = MODE == 1 ? s_hi : 0;
  f4 lw[FT], lb[FT];
  load_ln<FT>(a, h, lw, lb);
  Tile cdW1[FT][HT], cdW2[HT][FT];
  zero(cdW1);
  zero(cdW2);
  f4 db2T[FT], dlnw[FT], dlnb[FT];
#pragma unroll
  for (int c = 0; c < FT; ++c) db2T[c] = dlnw[c] = dlnb[c] = f4{0.f, 0.f, 0.f, 0.f};
  lds_order();
  if (l < FF) sdb1[l] = 0.f;
  lds_order();
  const float* states = a.saved + chain * a.per_chain + a.states;

  for (int s = s_hi; s >= s_lo; --s) {
    const float* S = states + (size_t)s * a.state;
    float* hs = MODE == 0 ? nullptr : a.hand + ((size_t)chain * NC + s) * HS::FLOATS;
    Tile cW1[FT][HT], cW2[HT][FT];
    f4 b2T[FT];
    load_mlp_state<FT, HT>(S, S + F * FF, S + F * FF + FF, S + F * FF + FF + FF * F, cW1, cW2, sb1, b2T);
    const size_t row0 = ((size_t)chain * NC + s) * K;
    SmallInputs<T, KT, FT> in;
    in.load(a, row0);
    float b1n[HT], db1n[HT];
    f4 b1T[HT];
    lds_order();
#pragma unroll
    for (int o = 0; o < HT; ++o) {
      b1n[o] = sb1[16 * o + n];
      b1T[o] = *reinterpret_cast<const f4*>(sb1 + 16 * o + 4 * g);
      db1n[o] = sdb1[16 * o + n];  // dL/db1 of the state after s
    }
    lds_order();
    float rs2[KT], rsb[KT];
    Tile outT[FT][KT];  // (MODE 1: the normalised Z2b rows)
    mlp_step<T, KT, FT, HT, true, RO, P, MODE != 1, MODE == 1>(in, cW1, cW2, b1n, b1T, b2T, lw, lb, a.eps, st, pk,
                                                              rs2, rsb, outT);
    Frag<T> fW2[HT][FT], fW2t[FT][HT], fW1[FT][HT];
    frags_t<T>(cW2, fW2t);
    {
      Tile w2T[FT][HT], w1T[HT][FT];
      tr(cW2, w2T, st);
      frags_t<T>(w2T, fW2);
      tr(cW1, w1T, st);
      frags_t<T>(w1T, fW1);
    }
    f4 db2c[FT];  // this mini-batch's db2 terms (token-layout form, per lane)
    Tile dg1[KT][HT];
    // ---- (1) through the update W' = W - X^T diag(e) G, b' = b - G^T e
    if constexpr (UP) {
      Frag<T> fdW1t[HT][FT], fdW2t[FT][HT];
      frags_t<T>(cdW1, fdW1t);
      frags_t<T>(cdW2, fdW2t);
      // t1 = XK dW1' + db1' (row): dg1 = -e t1, de = -sum t1 G1
      f4 deR[KT];
      {
        Tile t1[KT][HT], g1[KT][HT];
#pragma unroll
        for (int i = 0; i < KT; ++i)
#pragma unroll
          for (int o = 0; o < HT; ++o) t1[i][o].v = f4{db1n[o], db1n[o], db1n[o], db1n[o]};
        gemm<KT, HT, FT>(t1, in.k, fdW1t);
        unpark(pk + P::G1, g1);
#pragma unroll
        for (int i = 0; i < KT; ++i) {
          f4 d = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int o = 0; o < HT; ++o) {
            d -= t1[i][o].v * g1[i][o].v;
            dg1[i][o].v = -in.e4[i] * t1[i][o].v;
          }
          deR[i] = sum_row16_4(d);
        }
        // dxk = -e (G1 dW1'^T) (token)
        Tile dW1T[HT][FT], g1T[HT][KT], dxkT[FT][KT];
        tr(cdW1, dW1T, st);
        tr(g1, g1T, st);
        Frag<T> fdW1[FT][HT], fG1[KT][HT];
        frags_t<T>(dW1T, fdW1);
        frags_t<T>(g1T, fG1);
        zero(dxkT);
        gemm<FT, KT, HT>(dxkT, fdW1, fG1);
#pragma unroll
        for (int c = 0; c < FT; ++c)
#pragma unroll
          for (int i = 0; i < KT; ++i) dxkT[c][i].v *= -in.eT[i];
        park(pk + P::DXKT, dxkT);
      }
      // t2 = X2 dW2' + db2' (token): dg2 = -e t2, de -= sum t2 G2
      float deT[KT];
      {
        Tile x2[KT][HT], x2T[HT][KT], g2T[FT][KT];
        unpark(pk + P::X2, x2);
        tr(x2, x2T, st);
        unpark(pk + P::G2T, g2T);
        Frag<T> fX2[KT][HT], fG2[KT][FT];
        frags_t<T>(x2T, fX2);
        frags_t<T>(g2T, fG2);
        Tile t2T[FT][KT];
#pragma unroll
        for (int c = 0; c < FT; ++c)
#pragma unroll
          for (int i = 0; i < KT; ++i) t2T[c][i].v = db2T[c];
        gemm<FT, KT, HT>(t2T, fdW2t, fX2);
#pragma unroll
        for (int i = 0; i < KT; ++i) {
          float d = 0.f;
#pragma unroll
          for (int c = 0; c < FT; ++c) {
            d -= hsum(t2T[c][i].v * g2T[c][i].v);
            t2T[c][i].v *= -in.eT[i];  // dg2
          }
          deT[i] = sum_col4(d);
        }
        park(pk + P::DG2T, t2T);
        // dx2 = -e (G2 dW2'^T) (row)
        Tile dW2T[FT][HT], dx2[KT][HT];
        tr(cdW2, dW2T, st);
        Frag<T> fdW2[HT][FT];
        frags_t<T>(dW2T, fdW2);
        zero(dx2);
        gemm<KT, HT, FT>(dx2, fG2, fdW2);
#pragma unroll
        for (int i = 0; i < KT; ++i)
#pragma unroll
          for (int o = 0; o < HT; ++o) dx2[i][o].v *= -in.e4[i];
        park(pk + P::DX2, dx2);
      }
      lds_order();
#pragma unroll
      for (int i = 0; i < KT; ++i)
        if (n == 0) *reinterpret_cast<f4*>(sde + 16 * i + 4 * g) = deR[i];
      lds_order();
#pragma unroll
      for (int i = 0; i < KT; ++i)
        if (g == 0) sde[16 * i + n] += deT[i];
      lds_order();
    } else {
      // the readout path alone: its terms start from zero
      zero(dg1);
      lds_order();
      if (l < K) sde[l] = 0.f;
      lds_order();
    }
    f4 db1cT[HT];  // this mini-batch's db1 terms from the token layout
    Frag<T> fXKt[FT][KT];
    if constexpr (RO) {
    // ---- (2) output LayerNorm: out = XQ + ln_w xhb + ln_b; dXQ starts as dout
    Tile dz2bT[FT][KT], dxqT[FT][KT];
    {
      const T* DO = static_cast<const T*>(a.dout) + row0 * F;
      Tile xhbT[FT][KT];
      if constexpr (MODE == 1) {
#pragma unroll
        for (int c = 0; c < FT; ++c)
#pragma unroll
          for (int i = 0; i < KT; ++i) xhbT[c][i] = outT[c][i];
      } else {
        unpark(pk + P::XHBT, xhbT);
      }
#pragma unroll
      for (int c = 0; c < FT; ++c) db2c[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        f4 dv[FT], xb[FT], dz[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          dv[c] = frag_to_f4(load_frag(DO + 16 * i * F, F, 16 * c));
          dxqT[c][i].v = dv[c];
          xb[c] = xhbT[c][i].v;
        }
        ln_out_bwd<FT>(dv, xb, lw, rsb[i], dz, dlnw, dlnb);
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          dz2bT[c][i].v = dz[c];
          db2c[c] += dz[c];
        }
      }
    }
    // ---- (3) Z2b = X2b W2 + b2 - (eta (A2 + 1)) G2, A2 = X2b X2^T
    Tile dz1bT[HT][KT];
    {
      Frag<T> fdz2b[KT][FT], fdz2bt[FT][KT];
      frags_t<T>(dz2bT, fdz2b);
      {
        Tile dz2bR[KT][FT];
        tr(dz2bT, dz2bR, st);
        frags_t<T>(dz2bR, fdz2bt);
      }
      Frag<T> fX2b[KT][HT], fX2bt[HT][KT];
      {
        Tile x2bT[HT][KT], x2bR[KT][HT];
        unpark(pk + P::X2BT, x2bT);
        frags_t<T>(x2bT, fX2b);
        tr(x2bT, x2bR, st);
        frags_t<T>(x2bR, fX2bt);
      }
      gemm<HT, FT, KT>(cdW2, fX2bt, fdz2bt);  // dW2 += X2b^T dz2b
      Tile dx2bT[HT][KT];
      zero(dx2bT);
      gemm<HT, KT, FT>(dx2bT, fW2, fdz2b);  // dx2b = dz2b W2^T (token)
      Tile dA2[KT][KT];
      {
        // -dC2 = G2 dz2b^T; A2 + 1
        Tile dm[KT][KT], ap[KT][KT];
        {
          Frag<T> fG2[KT][FT];
          Tile g2T[FT][KT];
          unpark(pk + P::G2T, g2T);
          frags_t<T>(g2T, fG2);
          zero(dm);
          gemm<KT, KT, FT>(dm, fG2, fdz2b);
        }
        {
          Frag<T> fX2[KT][HT];
          Tile x2[KT][HT], x2T[HT][KT];
          unpark(pk + P::X2, x2);
          tr(x2, x2T, st);
          frags_t<T>(x2T, fX2);
          zero(ap);
          gemm<KT, KT, HT>(ap, fX2, fX2b);
        }
        // deta = dC2 (A2 + 1)
        {
          Tile de[KT][KT];
#pragma unroll
          for (int j = 0; j < KT; ++j)
#pragma unroll
            for (int i = 0; i < KT; ++i) de[j][i].v = -dm[j][i].v * (ap[j][i].v + 1.0f);
          park(pk + P::DETA, de);
        }
        // dA2 = dC2 eta; -C2 = -eta (A2 + 1) in the row layout for dg2 += -(C2^T dz2b)
        {
          f4 eta[KT][KT];
          in.eta(eta);
#pragma unroll
          for (int j = 0; j < KT; ++j)
#pragma unroll
            for (int i = 0; i < KT; ++i) {
              dA2[j][i].v = -dm[j][i].v * eta[i][j];
              ap[j][i].v = -(eta[i][j] * (ap[j][i].v + 1.0f));
            }
        }
        Tile c2R[KT][KT];
        tr(ap, c2R, st);
        Frag<T> fnC2t[KT][KT];
        frags_t<T>(c2R, fnC2t);
        Tile dg2T[FT][KT];
        if constexpr (MODE == 1) {
          zero(dg2T);
          gemm<FT, KT, KT>(dg2T, fdz2bt, fnC2t);
          hand_store(hs + HS::DG2T, dg2T);
        } else {
          unpark(pk + P::DG2T, dg2T);
          gemm<FT, KT, KT>(dg2T, fdz2bt, fnC2t);
          park(pk + P::DG2T, dg2T);
        }
      }
      // dx2b += dA2 X2 (token); dx2 += dA2^T X2b (row)
      {
        Frag<T> fdA2[KT][KT], fX2t[HT][KT];
        frags_t<T>(dA2, fdA2);
        {
          Tile x2[KT][HT];
          unpark(pk + P::X2, x2);
          frags_t<T>(x2, fX2t);
        }
        gemm<HT, KT, KT>(dx2bT, fX2t, fdA2);
        Tile dA2R[KT][KT];
        tr(dA2, dA2R, st);
        Frag<T> fdA2t[KT][KT];
        frags_t<T>(dA2R, fdA2t);
        Tile dx2[KT][HT];
        if constexpr (MODE == 1) {
          zero(dx2);
          gemm<KT, HT, KT>(dx2, fdA2t, fX2bt);
          hand_store(hs + HS::DX2, dx2);
        } else {
          unpark(pk + P::DX2, dx2);
          gemm<KT, HT, KT>(dx2, fdA2t, fX2bt);
          park(pk + P::DX2, dx2);
        }
      }
      {
        Tile db1T[HT][KT];
        unpark(pk + P::DB1T, db1T);
#pragma unroll
        for (int o = 0; o < HT; ++o)
#pragma unroll
          for (int i = 0; i < KT; ++i) dz1bT[o][i].v = dx2bT[o][i].v * db1T[o][i].v;
      }
    }
    // ---- (4) Z1b = XQ W1 + b1 - (eta (A1 + 1)) G1, A1 = XQ XK^T
    {
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        f4 d = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < KT; ++i) d += dz1bT[o][i].v;
        db1cT[o] = sum_row16_4(d);
      }
      Frag<T> fdz1b[KT][HT], fdz1bt[HT][KT];
      frags_t<T>(dz1bT, fdz1b);
      {
        Tile dz1bR[KT][HT];
        tr(dz1bT, dz1bR, st);
        frags_t<T>(dz1bR, fdz1bt);
      }
      gemm<FT, KT, HT>(dxqT, fW1, fdz1b);  // dxq += dz1b W1^T (token)
      Frag<T> fXQt[FT][KT];
      {
        Tile xT[FT][KT], xR[KT][FT];
        tiles_of<T>(in.q, xT);
        tr(xT, xR, st);
        frags_t<T>(xR, fXQt);
        tiles_of<T>(in.k, xT);
        tr(xT, xR, st);
        frags_t<T>(xR, fXKt);
      }
      gemm<FT, HT, KT>(cdW1, fXQt, fdz1bt);  // dW1 += XQ^T dz1b
      Tile dA1[KT][KT];
      {
        // -dC1 = G1 dz1b^T; A1 + 1
        Tile dm[KT][KT], ap[KT][KT];
        {
          Frag<T> fG1[KT][HT];
          Tile g1[KT][HT], g1T[HT][KT];
          unpark(pk + P::G1, g1);
          tr(g1, g1T, st);
          frags_t<T>(g1T, fG1);
          zero(dm);
          gemm<KT, KT, HT>(dm, fG1, fdz1b);
        }
        zero(ap);
        gemm<KT, KT, FT>(ap, in.k, in.q);
        {
          Tile de[KT][KT];
          unpark(pk + P::DETA, de);
#pragma unroll
          for (int j = 0; j < KT; ++j)
#pragma unroll
            for (int i = 0; i < KT; ++i) de[j][i].v -= dm[j][i].v * (ap[j][i].v + 1.0f);
          store_deta<T, KT>(a, row0, de, sde);
        }
        {
          f4 eta[KT][KT];
          in.eta(eta);
#pragma unroll
          for (int j = 0; j < KT; ++j)
#pragma unroll
            for (int i = 0; i < KT; ++i) {
              dA1[j][i].v = -dm[j][i].v * eta[i][j];
              ap[j][i].v = -(eta[i][j] * (ap[j][i].v + 1.0f));
            }
        }
        // dg1 += -(C1^T dz1b) (row)
        Tile c1R[KT][KT];
        tr(ap, c1R, st);
        Frag<T> fnC1t[KT][KT];
        frags_t<T>(c1R, fnC1t);
        gemm<KT, HT, KT>(dg1, fnC1t, fdz1bt);
      }
      // dxq += dA1 XK (token); dxk += dA1^T XQ (token)
      {
        Frag<T> fdA1[KT][KT], fdA1t[KT][KT];
        frags_t<T>(dA1, fdA1);
        gemm<FT, KT, KT>(dxqT, fXKt, fdA1);
        store_rows<T, KT, FT>(a.dXQ, row0, dxqT);
        Tile dA1R[KT][KT];
        tr(dA1, dA1R, st);
        frags_t<T>(dA1R, fdA1t);
        Tile dxkT[FT][KT];
        if constexpr (MODE == 1) {
          zero(dxkT);
          gemm<FT, KT, KT>(dxkT, fXQt, fdA1t);
          hand_store(hs + HS::DXKT, dxkT);
        } else {
          unpark(pk + P::DXKT, dxkT);
          gemm<FT, KT, KT>(dxkT, fXQt, fdA1t);
          park(pk + P::DXKT, dxkT);
        }
      }
    }
    }  // RO
    if constexpr (MODE == 1) {
      // the handoff: this mini-batch's readout-path terms (dG2, dX2 and dXK
      // went there from phases (3) and (4))
      hand_store(hs + HS::DG1, dg1);
      hand_store(hs + HS::DW1, cdW1);
      hand_store(hs + HS::DW2, cdW2);
      hand_store4(hs + HS::DB1T, db1cT);
      hand_store4(hs + HS::DB2C, db2c);
      hand_store4(hs + HS::DLNW, dlnw);
      hand_store4(hs + HS::DLNB, dlnb);
    } else if constexpr (MODE == 2) {
      // the readout path's terms from the handoff, added after (1)
      Tile t[FT][KT], r[KT][HT];
      hand_add(hs + HS::DG1, dg1);
      unpark(pk + P::DG2T, t);
      hand_add(hs + HS::DG2T, t);
      park(pk + P::DG2T, t);
      unpark(pk + P::DXKT, t);
      hand_add(hs + HS::DXKT, t);
      park(pk + P::DXKT, t);
      unpark(pk + P::DX2, r);
      hand_add(hs + HS::DX2, r);
      park(pk + P::DX2, r);
      hand_add(hs + HS::DW1, cdW1);
      hand_add(hs + HS::DW2, cdW2);
      hand_load4(hs + HS::DB1T, db1cT);
      hand_load4(hs + HS::DB2C, db2c);
      f4 x[FT];
      hand_load4(hs + HS::DLNW, x);
#pragma unroll
      for (int c = 0; c < FT; ++c) dlnw[c] += x[c];
      hand_load4(hs + HS::DLNB, x);
#pragma unroll
      for (int c = 0; c < FT; ++c) dlnb[c] += x[c];
      // XK's transposed operand frags (phase (4) forms them in MODE 0)
      {
        Tile xT[FT][KT], xR[KT][FT];
        tiles_of<T>(in.k, xT);
        tr(xT, xR, st);
        frags_t<T>(xR, fXKt);
      }
      // the update term of deta's last row, which the readout launch left out
      lds_order();
      if (l < K) add_deta_last_row<T>(a, row0, K, l, sde[l]);
      lds_order();
    }
    if constexpr (UP) {
    // ---- (5) G1 = P1 gelu'(Z1): dp = dg1 gelu'(Z1), dz1 = dg1 P1 gelu''(Z1)
    Tile dz1[KT][HT];
    {
      Tile dp[KT][HT];
      {
        Tile d1[KT][HT], pdd[KT][HT];
        unpark(pk + P::D1, d1);
        unpark(pk + P::PDD, pdd);
#pragma unroll
        for (int i = 0; i < KT; ++i)
#pragma unroll
          for (int o = 0; o < HT; ++o) {
            dp[i][o].v = dg1[i][o].v * d1[i][o].v;
            dz1[i][o].v = dg1[i][o].v * pdd[i][o].v;
          }
      }
      // dg2 += dp W2 (token); dW2 += dp^T G2
      Tile dpT[HT][KT];
      tr(dp, dpT, st);
      Frag<T> fdp[KT][HT], fdpt[HT][KT], fG2t[FT][KT];
      frags_t<T>(dpT, fdp);
      frags_t<T>(dp, fdpt);
      Tile dg2T[FT][KT];
      unpark(pk + P::DG2T, dg2T);
      gemm<FT, KT, HT>(dg2T, fW2t, fdp);
      park(pk + P::DG2T, dg2T);
      {
        Tile g2T[FT][KT], g2R[KT][FT];
        unpark(pk + P::G2T, g2T);
        tr(g2T, g2R, st);
        frags_t<T>(g2R, fG2t);
      }
      gemm<HT, FT, KT>(cdW2, fdpt, fG2t);
    }
    // ---- (6) G2 = ln_fused_l2_bwd(Z2, XV - XK): its backward (token)
    Tile dz2T[FT][KT], dxkT[FT][KT];
    {
      Tile xh2T[FT][KT], g2T[FT][KT], dg2T[FT][KT], dxvT[FT][KT];
      unpark(pk + P::XH2T, xh2T);
      unpark(pk + P::G2T, g2T);
      unpark(pk + P::DG2T, dg2T);
      unpark(pk + P::DXKT, dxkT);
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        f4 xh[FT], qv[FT], G[FT], tg[FT], dz[FT], dt[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          xh[c] = xh2T[c][i].v;
          qv[c] = dg2T[c][i].v;
          G[c] = g2T[c][i].v;
          tg[c] = frag_to_f4(in.v[i][c]) - frag_to_f4(in.k[i][c]);
        }
        ln_l2_bwd<FT>(xh, qv, G, tg, lw, lb, rs2[i], dz, dt, dlnw, dlnb);
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          dxvT[c][i].v = dt[c];
          dxkT[c][i].v -= dt[c];
          dz2T[c][i].v = dz[c];
          db2c[c] += dz[c];
        }
      }
      store_rows<T, KT, FT>(a.dXV, row0, dxvT);
    }
    // ---- (7) Z2 = X2 W2 + b2, X2 = gelu(Z1), Z1 = XK W1 + b1
    float db1c[HT];  // this mini-batch's db1 terms in feature order n (row-layout sums)
    {
      Frag<T> fdz2[KT][FT], fdz2t[FT][KT], fX2t[HT][KT];
      frags_t<T>(dz2T, fdz2);
      {
        Tile dz2R[KT][FT];
        tr(dz2T, dz2R, st);
        frags_t<T>(dz2R, fdz2t);
      }
      Tile dx2[KT][HT];
      unpark(pk + P::DX2, dx2);
      gemm<KT, HT, FT>(dx2, fdz2, fW2);  // dx2 += dz2 W2^T
      {
        Tile x2[KT][HT];
        unpark(pk + P::X2, x2);
        frags_t<T>(x2, fX2t);
      }
      gemm<HT, FT, KT>(cdW2, fX2t, fdz2t);  // dW2 += X2^T dz2
      {
        Tile d1[KT][HT];
        unpark(pk + P::D1, d1);
#pragma unroll
        for (int i = 0; i < KT; ++i)
#pragma unroll
          for (int o = 0; o < HT; ++o) dz1[i][o].v += dx2[i][o].v * d1[i][o].v;
      }
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < KT; ++i) d += hsum(dz1[i][o].v);
        db1c[o] = sum_col4(d);
      }
      Tile dz1T[HT][KT];
      tr(dz1, dz1T, st);
      Frag<T> fdz1[KT][HT], fdz1t[HT][KT];
      frags_t<T>(dz1T, fdz1);
      frags_t<T>(dz1, fdz1t);
      gemm<FT, KT, HT>(dxkT, fW1, fdz1);    // dxk += dz1 W1^T
      gemm<FT, HT, KT>(cdW1, fXKt, fdz1t);  // dW1 += XK^T dz1
      store_rows<T, KT, FT>(a.dXK, row0, dxkT);
    }
    // ---- bias gradients: db entering the mini-batch = db' + its terms
#pragma unroll
    for (int c = 0; c < FT; ++c) db2T[c] += sum_row16_4(db2c[c]);
    lds_order();
#pragma unroll
    for (int o = 0; o < HT; ++o)
      if (g == 0) sdb1[16 * o + n] = db1n[o] + db1c[o];
    lds_order();
#pragma unroll
    for (int o = 0; o < HT; ++o)
      if (n == 0) *reinterpret_cast<f4*>(sdb1 + 16 * o + 4 * g) += db1cT[o];
    lds_order();
    }  // UP
  }
  if constexpr (MODE == 1) return;
  // the initial state's gradient and the LayerNorm parameters' (per chain)
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < HT; ++o) store_tile(a.dW1 + chain * F * FF, FF, 16 * i, 16 * o, cdW1[i][o]);
#pragma unroll
  for (int o = 0; o < HT; ++o)
#pragma unroll
    for (int c = 0; c < FT; ++c) store_tile(a.dW2 + chain * FF * F, F, 16 * o, 16 * c, cdW2[o][c]);
  lds_order();
  if (l < FF) a.db1[chain * FF + l] = sdb1[l];
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    const f4 w = sum_row16_4(dlnw[c]), b = sum_row16_4(dlnb[c]);
    if (n == 0) {
      store4(a.db2 + chain * F + 16 * c + 4 * g, db2T[c]);
      store4(a.dln_w + chain * F + 16 * c + 4 * g, w);
      store4(a.dln_b + chain * F + 16 * c + 4 * g, b);
    }
  }
}

// ---------------------------------------------------------------- TTT-Linear
//
// Per mini-batch (ops/ttt_linear.py:8-54), everything token-major but the
// state: Z = XK W + b, G = ln_fused_l2_bwd(Z, XV - XK) (also in the row
// layout), Zb = XQ W + b - (eta (A1 + 1)) G, out = XQ + LN(Zb).
template <int KT, int FT, bool FULL> struct LinPark {
  static constexpr int TF = FT * KT * 256;
  static constexpr int KK = KT * KT * 256;
  static constexpr int GT = 0;                          // G (token)
  static constexpr int XHT = GT + TF;                   // backward only: normalised Z (token)
  static constexpr int XHBT = XHT + (FULL ? TF : 0);    // normalised Zb (token)
  static constexpr int A1P = XHBT + (FULL ? TF : 0);    // A1 + 1, tiles [t'][t]
  static constexpr int FLOATS = A1P + (FULL ? KK : 0);
};

template <typename T, int KT, int FT, bool FULL>
__device__ __forceinline__ void lin_step(const SmallInputs<T, KT, FT>& in, const Tile (&W)[FT][FT], const f4 (&bT)[FT],
                                         const f4 (&lw)[FT], const f4 (&lb)[FT], float eps, float* st, float* pk,
                                         float (&rs)[KT], float (&rsb)[KT], Tile (&outT)[FT][KT]) {
  using P = LinPark<KT, FT, FULL>;
  Frag<T> fWt[FT][FT];
  frags_t<T>(W, fWt);
  Frag<T> fGt[FT][KT];
  {
    Tile zT[FT][KT];
#pragma unroll
    for (int c = 0; c < FT; ++c)
#pragma unroll
      for (int i = 0; i < KT; ++i) zT[c][i].v = bT[c];
    gemm<FT, KT, FT>(zT, fWt, in.k);
    Tile gT[FT][KT], xhT[FT][KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) {
      f4 z[FT], tg[FT], xh[FT], G[FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        z[c] = zT[c][i].v;
        tg[c] = frag_to_f4(in.v[i][c]) - frag_to_f4(in.k[i][c]);
      }
      ln_l2_fwd<FT>(z, tg, lw, lb, eps, xh, G, rs[i]);
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        gT[c][i].v = G[c];
        xhT[c][i].v = xh[c];
      }
    }
    park(pk + P::GT, gT);
    if constexpr (FULL) park(pk + P::XHT, xhT);
    Tile gR[KT][FT];
    tr(gT, gR, st);
    frags_t<T>(gR, fGt);
  }
  f4 eta[KT][KT];
  in.eta(eta);
  Frag<T> fnC1[KT][KT];
  {
    Tile a1T[KT][KT];
    zero(a1T);
    gemm<KT, KT, FT>(a1T, in.k, in.q);
#pragma unroll
    for (int j = 0; j < KT; ++j)
#pragma unroll
      for (int i = 0; i < KT; ++i) a1T[j][i].v += 1.0f;
    if constexpr (FULL) park(pk + P::A1P, a1T);
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
      for (int j = 0; j < KT; ++j) fnC1[i][j] = to_frag<T>(-(eta[i][j] * a1T[j][i].v));
  }
  Tile zbT[FT][KT];
#pragma unroll
  for (int c = 0; c < FT; ++c)
#pragma unroll
    for (int i = 0; i < KT; ++i) zbT[c][i].v = bT[c];
  gemm<FT, KT, FT>(zbT, fWt, in.q);
  gemm<FT, KT, KT>(zbT, fGt, fnC1);
  Tile xhbT[FT][KT];
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    f4 z[FT];
#pragma unroll
    for (int c = 0; c < FT; ++c) z[c] = zbT[c][i].v;
    float mu;
    ln_stats<FT>(z, eps, mu, rsb[i]);
#pragma unroll
    for (int c = 0; c < FT; ++c) {
      xhbT[c][i].v = (z[c] - mu) * rsb[i];
      outT[c][i].v = frag_to_f4(in.q[i][c]) + lw[c] * xhbT[c][i].v + lb[c];
    }
  }
  if constexpr (FULL) park(pk + P::XHBT, xhbT);
}

template <int FT>
__device__ __forceinline__ void load_lin_state(const float* W, const float* b, Tile (&cW)[FT][FT], f4 (&bT)[FT]) {
  constexpr int F = 16 * FT;
  const int g = lane_id() >> 4;
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < FT; ++o) cW[i][o] = load_tile(W, F, 16 * i, 16 * o);
#pragma unroll
  for (int c = 0; c < FT; ++c) bT[c] = load4(b + 16 * c + 4 * g);
}
template <int FT>
__device__ __forceinline__ void store_lin_state(float* W, float* b, const Tile (&cW)[FT][FT], const f4 (&bT)[FT]) {
  constexpr int F = 16 * FT;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  if (W != nullptr) {
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) store_tile(W, F, 16 * i, 16 * o, cW[i][o]);
  }
  if (b != nullptr && n == 0) {
#pragma unroll
    for (int c = 0; c < FT; ++c) store4(b + 16 * c + 4 * g, bT[c]);
  }
}

template <typename T, int KT, int FT>
__global__ __launch_bounds__(64) void small_lin_fwd_kernel(SmallArgs a) {
  constexpr int K = 16 * KT, F = 16 * FT;
  using P = LinPark<KT, FT, false>;
  __shared__ __align__(16) float st[kStage];
  __shared__ __align__(16) float pk[P::FLOATS];
  const size_t chain = blockIdx.x;
  const int h = (int)(chain % a.H), NC = a.NC;
  Tile cW[FT][FT];
  f4 bT[FT];
  load_lin_state<FT>(a.W1_init + chain * F * F, a.b1_init + chain * F, cW, bT);
  f4 lw[FT], lb[FT];
  load_ln<FT>(a, h, lw, lb);
  float* states = a.saved + chain * a.per_chain + a.states;
  for (int s = 0; s < NC; ++s) {
    {
      float* S = states + (size_t)s * a.state;
      store_lin_state<FT>(S, S + F * F, cW, bT);
    }
    if (a.ckpt[0] != nullptr && s % a.G == 0) {
      const size_t k = chain * a.NK + s / a.G;
      store_lin_state<FT>(a.ckpt[0] + k * F * F, a.ckpt[1] ? a.ckpt[1] + k * F : nullptr, cW, bT);
    }
    const size_t row0 = ((size_t)chain * NC + s) * K;
    SmallInputs<T, KT, FT> in;
    in.load(a, row0);
    {
      float rs[KT], rsb[KT];
      Tile outT[FT][KT];
      lin_step<T, KT, FT, false>(in, cW, bT, lw, lb, a.eps, st, pk, rs, rsb, outT);
      store_rows<T, KT, FT>(a.out, row0, outT);
    }
    // W -= XK^T diag(e) G, b -= G^T e (ops/ttt_linear.py:39-41)
    {
      Tile xkT[FT][KT], xkR[KT][FT], gT[FT][KT], gR[KT][FT];
      tiles_of<T>(in.k, xkT);
      tr(xkT, xkR, st);
      unpark(pk + P::GT, gT);
      tr(gT, gR, st);
      Frag<T> fXKt[FT][KT], fnGe[FT][KT];
      frags_t<T>(xkR, fXKt);
      f4 ne[KT];
#pragma unroll
      for (int i = 0; i < KT; ++i) ne[i] = -in.e4[i];
      frags_t_scaled<T>(gR, ne, fnGe);
      gemm<FT, FT, KT>(cW, fXKt, fnGe);
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        f4 d = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < KT; ++i) d += in.eT[i] * gT[c][i].v;
        bT[c] -= sum_row16_4(d);
      }
    }
  }
  if (a.last[0] != nullptr) store_lin_state<FT>(a.last[0] + chain * F * F, a.last[1] + chain * F, cW, bT);
}

template <typename T, int KT, int FT>
__global__ __launch_bounds__(64) void small_lin_bwd_kernel(SmallArgs a) {
  constexpr int K = 16 * KT, F = 16 * FT;
  using P = LinPark<KT, FT, true>;
  __shared__ __align__(16) float st[kStage];
  __shared__ __align__(16) float pk[P::FLOATS];
  __shared__ __align__(16) float sde[K];
  const size_t chain = blockIdx.x;
  const int h = (int)(chain % a.H), NC = a.NC;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  f4 lw[FT], lb[FT];
  load_ln<FT>(a, h, lw, lb);
  Tile cdW[FT][FT];
  zero(cdW);
  f4 dbT[FT], dlnw[FT], dlnb[FT];
#pragma unroll
  for (int c = 0; c < FT; ++c) dbT[c] = dlnw[c] = dlnb[c] = f4{0.f, 0.f, 0.f, 0.f};
  const float* states = a.saved + chain * a.per_chain + a.states;
  for (int s = NC - 1; s >= 0; --s) {
    const float* S = states + (size_t)s * a.state;
    Tile cW[FT][FT];
    f4 bT[FT];
    load_lin_state<FT>(S, S + F * F, cW, bT);
    const size_t row0 = ((size_t)chain * NC + s) * K;
    SmallInputs<T, KT, FT> in;
    in.load(a, row0);
    float rs[KT], rsb[KT];
    {
      Tile outT[FT][KT];
      lin_step<T, KT, FT, true>(in, cW, bT, lw, lb, a.eps, st, pk, rs, rsb, outT);
    }
    Frag<T> fW[FT][FT];
    {
      Tile wT[FT][FT];
      tr(cW, wT, st);
      frags_t<T>(wT, fW);
    }
    Tile dgT[FT][KT], dxkT[FT][KT];
    f4 dbc[FT];
    // ---- (1) through the update: t = XK dW' + db', dg = -e t, de = -sum t G; dxk = -e (G dW'^T)
    {
      Tile gT[FT][KT];
      unpark(pk + P::GT, gT);
      Frag<T> fdWt[FT][FT], fG[KT][FT];
      frags_t<T>(cdW, fdWt);
      frags_t<T>(gT, fG);
      Tile tT[FT][KT];
#pragma unroll
      for (int c = 0; c < FT; ++c)
#pragma unroll
        for (int i = 0; i < KT; ++i) tT[c][i].v = dbT[c];
      gemm<FT, KT, FT>(tT, fdWt, in.k);
      float deT[KT];
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        float d = 0.f;
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          d -= hsum(tT[c][i].v * gT[c][i].v);
          dgT[c][i].v = -in.eT[i] * tT[c][i].v;
        }
        deT[i] = sum_col4(d);
      }
      lds_order();
#pragma unroll
      for (int i = 0; i < KT; ++i)
        if (g == 0) sde[16 * i + n] = deT[i];
      lds_order();
      Tile dWT[FT][FT];
      tr(cdW, dWT, st);
      Frag<T> fdW[FT][FT];
      frags_t<T>(dWT, fdW);
      zero(dxkT);
      gemm<FT, KT, FT>(dxkT, fdW, fG);
#pragma unroll
      for (int c = 0; c < FT; ++c)
#pragma unroll
        for (int i = 0; i < KT; ++i) dxkT[c][i].v *= -in.eT[i];
    }
    // ---- (2) output LayerNorm; dXQ starts as dout
    Tile dzbT[FT][KT], dxqT[FT][KT];
    {
      const T* DO = static_cast<const T*>(a.dout) + row0 * F;
      Tile xhbT[FT][KT];
      unpark(pk + P::XHBT, xhbT);
#pragma unroll
      for (int c = 0; c < FT; ++c) dbc[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        f4 dv[FT], xb[FT], dz[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          dv[c] = frag_to_f4(load_frag(DO + 16 * i * F, F, 16 * c));
          dxqT[c][i].v = dv[c];
          xb[c] = xhbT[c][i].v;
        }
        ln_out_bwd<FT>(dv, xb, lw, rsb[i], dz, dlnw, dlnb);
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          dzbT[c][i].v = dz[c];
          dbc[c] += dz[c];
        }
      }
    }
    // ---- (3) Zb = XQ W + b - (eta (A1 + 1)) G
    Frag<T> fXKt[FT][KT];
    {
      Frag<T> fdzb[KT][FT], fdzbt[FT][KT], fXQt[FT][KT];
      frags_t<T>(dzbT, fdzb);
      {
        Tile r[KT][FT], xT[FT][KT];
        tr(dzbT, r, st);
        frags_t<T>(r, fdzbt);
        tiles_of<T>(in.q, xT);
        tr(xT, r, st);
        frags_t<T>(r, fXQt);
        tiles_of<T>(in.k, xT);
        tr(xT, r, st);
        frags_t<T>(r, fXKt);
      }
      gemm<FT, FT, KT>(cdW, fXQt, fdzbt);  // dW += XQ^T dzb
      gemm<FT, KT, FT>(dxqT, fW, fdzb);    // dxq += dzb W^T
      f4 eta[KT][KT];
      in.eta(eta);
      Tile dA1[KT][KT], detaT[KT][KT];
      {
        Frag<T> fG[KT][FT];
        {
          Tile gT[FT][KT];
          unpark(pk + P::GT, gT);
          frags_t<T>(gT, fG);
        }
        Tile ap[KT][KT];
        zero(dA1);
        gemm<KT, KT, FT>(dA1, fG, fdzb);  // -dC1 (token tiles [t'][t])
        unpark(pk + P::A1P, ap);
#pragma unroll
        for (int j = 0; j < KT; ++j)
#pragma unroll
          for (int i = 0; i < KT; ++i) {
            detaT[j][i].v = -dA1[j][i].v * ap[j][i].v;
            dA1[j][i].v = -dA1[j][i].v * eta[i][j];
          }
        Tile c1R[KT][KT];
#pragma unroll
        for (int j = 0; j < KT; ++j)
#pragma unroll
          for (int i = 0; i < KT; ++i) ap[j][i].v = -(eta[i][j] * ap[j][i].v);
        tr(ap, c1R, st);
        Frag<T> fnC1t[KT][KT];
        frags_t<T>(c1R, fnC1t);
        gemm<FT, KT, KT>(dgT, fdzbt, fnC1t);  // dg += -(C1^T dzb)
      }
      store_deta<T, KT>(a, row0, detaT, sde);
      {
        Frag<T> fdA1[KT][KT], fdA1t[KT][KT];
        frags_t<T>(dA1, fdA1);
        gemm<FT, KT, KT>(dxqT, fXKt, fdA1);  // dxq += dA1 XK
        Tile dA1R[KT][KT];
        tr(dA1, dA1R, st);
        frags_t<T>(dA1R, fdA1t);
        gemm<FT, KT, KT>(dxkT, fXQt, fdA1t);  // dxk += dA1^T XQ
      }
      store_rows<T, KT, FT>(a.dXQ, row0, dxqT);
    }
    // ---- (4) G = ln_fused_l2_bwd(Z, XV - XK): its backward
    Tile dzT[FT][KT];
    {
      Tile xhT[FT][KT], gT[FT][KT], dxvT[FT][KT];
      unpark(pk + P::XHT, xhT);
      unpark(pk + P::GT, gT);
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        f4 xh[FT], qv[FT], G[FT], tg[FT], dz[FT], dt[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          xh[c] = xhT[c][i].v;
          qv[c] = dgT[c][i].v;
          G[c] = gT[c][i].v;
          tg[c] = frag_to_f4(in.v[i][c]) - frag_to_f4(in.k[i][c]);
        }
        ln_l2_bwd<FT>(xh, qv, G, tg, lw, lb, rs[i], dz, dt, dlnw, dlnb);
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          dxvT[c][i].v = dt[c];
          dxkT[c][i].v -= dt[c];
          dzT[c][i].v = dz[c];
          dbc[c] += dz[c];
        }
      }
      store_rows<T, KT, FT>(a.dXV, row0, dxvT);
    }
    // ---- (5) Z = XK W + b
    {
      Frag<T> fdz[KT][FT], fdzt[FT][KT];
      frags_t<T>(dzT, fdz);
      Tile r[KT][FT];
      tr(dzT, r, st);
      frags_t<T>(r, fdzt);
      gemm<FT, KT, FT>(dxkT, fW, fdz);    // dxk += dz W^T
      gemm<FT, FT, KT>(cdW, fXKt, fdzt);  // dW += XK^T dz
      store_rows<T, KT, FT>(a.dXK, row0, dxkT);
    }
#pragma unroll
    for (int c = 0; c < FT; ++c) dbT[c] += sum_row16_4(dbc[c]);
  }
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < FT; ++o) store_tile(a.dW1 + chain * F * F, F, 16 * i, 16 * o, cdW[i][o]);
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    const f4 w = sum_row16_4(dlnw[c]), b = sum_row16_4(dlnb[c]);
    if (n == 0) {
      store4(a.db1 + chain * F + 16 * c + 4 * g, dbT[c]);
      store4(a.dln_w + chain * F + 16 * c + 4 * g, w);
      store4(a.dln_b + chain * F + 16 * c + 4 * g, b);
    }
  }
}

template <typename T, int KT> hipError_t launch_kt(const SmallArgs& a, int BH, bool mlp, bool bwd, hipStream_t s) {
  if (mlp) {
    if (bwd && a.hand != nullptr) {
      // two launches: the readout path of every (chain, mini-batch) at once, then the sweeps
      hipLaunchKernelGGL((small_mlp_bwd_kernel<T, KT, 2, 2, 1>), dim3(BH * a.NC), dim3(64), 0, s, a);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((small_mlp_bwd_kernel<T, KT, 2, 2, 2>), dim3(BH), dim3(64), 0, s, a);
    } else if (bwd) {
      hipLaunchKernelGGL((small_mlp_bwd_kernel<T, KT, 2, 2, 0>), dim3(BH), dim3(64), 0, s, a);
    } else {
      hipLaunchKernelGGL((small_mlp_fwd_kernel<T, KT, 2, 2>), dim3(BH), dim3(64), 0, s, a);
    }
  } else {
    if (bwd) hipLaunchKernelGGL((small_lin_bwd_kernel<T, KT, 2>), dim3(BH), dim3(64), 0, s, a);
    else hipLaunchKernelGGL((small_lin_fwd_kernel<T, KT, 2>), dim3(BH), dim3(64), 0, s, a);
  }
  return hipGetLastError();
}

template <typename T> hipError_t launch_t(const SmallArgs& a, int BH, int K, bool mlp, bool bwd, hipStream_t s) {
  switch (K) {
    case 16: return launch_kt<T, 1>(a, BH, mlp, bwd, s);
    case 32: return launch_kt<T, 2>(a, BH, mlp, bwd, s);
    case 48: return launch_kt<T, 3>(a, BH, mlp, bwd, s);
    case 64: return launch_kt<T, 4>(a, BH, mlp, bwd, s);
    default: return hipErrorInvalidValue;
  }
}

SmallArgs small_args(int B, int H, int NC, int K, int F, int FF, bool mlp, float* saved) {
  SmallArgs a{};
  const GenLayout L(K, F, FF, NC, mlp);
  a.saved = saved;
  a.per_chain = L.per_chain;
  a.states = L.states;
  a.state = L.state;
  a.H = H;
  a.NC = NC;
  (void)B;
  return a;
}

}  // namespace

bool small_shape_ok(int K, int F, int FF, bool mlp) {
  if (K < 16 || K > 16 * kSmallMaxKT || K % 16) return false;
  return F == 32 && (!mlp || FF == 32);
}

size_t small_mlp_bwd_hand_bytes(int B, int H, int NC, int K) {
  size_t per = 0;
  switch (K) {
    case 16: per = MlpBwdHand<1, 2, 2>::FLOATS; break;
    case 32: per = MlpBwdHand<2, 2, 2>::FLOATS; break;
    case 48: per = MlpBwdHand<3, 2, 2>::FLOATS; break;
    case 64: per = MlpBwdHand<4, 2, 2>::FLOATS; break;
    default: return 0;
  }
  return (size_t)B * H * NC * per * sizeof(float);
}

hipError_t launch_small_fwd(const GenFwdParams& q, int dtype, hipStream_t stream) {
  SmallArgs a = small_args(q.B, q.H, q.NC, q.K, q.F, q.FF, q.mlp, static_cast<float*>(q.saved));
  a.XQ = q.XQ;
  a.XK = q.XK;
  a.XV = q.XV;
  a.eta = q.eta;
  a.ln_w = q.ln_w;
  a.ln_b = q.ln_b;
  a.W1_init = q.W1_init;
  a.b1_init = q.b1_init;
  a.W2_init = q.W2_init;
  a.b2_init = q.b2_init;
  a.out = q.out;
  float* last[4] = {q.W1_last, q.b1_last, q.W2_last, q.b2_last};
  float* ckpt[4] = {q.W1_ckpt, q.b1_ckpt, q.W2_ckpt, q.b2_ckpt};
  float* memo[4] = {q.W1_memo, q.b1_memo, q.W2_memo, q.b2_memo};
  for (int i = 0; i < 4; ++i) {
    a.last[i] = last[i];
    a.ckpt[i] = ckpt[i];
    a.memo[i] = memo[i];
  }
  a.G = q.G;
  a.M = q.M;
  a.NK = (q.NC + q.G - 1) / q.G;
  a.NS = (q.NC + q.M - 1) / q.M;
  a.eta_rule = q.eta_rule;
  a.eps = q.eps;
  const int BH = q.B * q.H;
  if (dtype == TTT_DTYPE_BF16) return launch_t<__bf16>(a, BH, q.K, q.mlp, false, stream);
  if (dtype == TTT_DTYPE_F16) return launch_t<_Float16>(a, BH, q.K, q.mlp, false, stream);
  return launch_t<float>(a, BH, q.K, q.mlp, false, stream);
}

hipError_t launch_small_bwd(const GenBwdParams& q, int dtype, hipStream_t stream) {
  SmallArgs a = small_args(q.B, q.H, q.NC, q.K, q.F, q.FF, q.mlp, static_cast<float*>(q.saved));
  a.XQ = q.XQ;
  a.XK = q.XK;
  a.XV = q.XV;
  a.eta = q.eta;
  a.dout = q.dout;
  a.ln_w = q.ln_w;
  a.ln_b = q.ln_b;
  a.dXQ = q.dXQ;
  a.dXK = q.dXK;
  a.dXV = q.dXV;
  a.deta = q.deta;
  a.dW1 = q.dW1;
  a.db1 = q.db1;
  a.dW2 = q.dW2;
  a.db2 = q.db2;
  a.dln_w = q.dln_w;
  a.dln_b = q.dln_b;
  a.G = 1;
  a.M = 1;
  a.eta_rule = q.eta_rule;
  a.eps = q.eps;
  // the two-launch MLP backward when the workspace holds its handoff
  const size_t hand = q.mlp ? small_mlp_bwd_hand_bytes(q.B, q.H, q.NC, q.K) : 0;
  a.hand = hand > 0 && q.ws != nullptr && q.ws_bytes >= hand ? static_cast<float*>(q.ws) : nullptr;
  const int BH = q.B * q.H;
  if (dtype == TTT_DTYPE_BF16) return launch_t<__bf16>(a, BH, q.K, q.mlp, true, stream);
  if (dtype == TTT_DTYPE_F16) return launch_t<_Float16>(a, BH, q.K, q.mlp, true, stream);
  return launch_t<float>(a, BH, q.K, q.mlp, true, stream);
}

}  // namespace ttt
