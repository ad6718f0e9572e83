// General-shape TTT inner loops (Linear and MLP) on gfx950: any mini-batch
// size K, head dim F and hidden width FF that are multiples of 16 (K <= 64,
// F <= 256, FF <= 1024), for the shapes the specialised kernels do not take
// (those hold K = 16 and F in {32, 64} in registers, FF in {64, 128, 256}).
// This is what the reference's own model configuration needs: TTTMLP sets
// FF = F (ttt_layer.py:427-430) and ModelConfig defaults to K = 64 with
// F = 32 (forecast.py:33-44).
//
// One workgroup of 256 threads per (batch, head) chain walks the mini-batches
// in order (ops/ttt_linear.py:8-54, ops/ttt_mlp.py:9-67, dual form with the
// full K x K eta).  All per-mini-batch matrices live in an fp32 scratch area
// of the chain inside the caller's `saved` buffer (L2-resident for the small
// shapes); every product is a cooperative fp32 GEMM in 4 x 4 register blocks,
// every LayerNorm a row pass, with a workgroup barrier between dependent
// steps.  The forward also stores the state entering every mini-batch there,
// so the backward visits the mini-batches in reverse, recomputes one
// mini-batch's forward values from its stored state and applies the
// hand-derived gradient of that mini-batch (chain rule through the update,
// the output LayerNorm, both dual-form attention products, the GELU and its
// derivative, and the LayerNorm fused with the L2 loss).  Everything is fp32
// whatever the activation type; the activations are converted on load.
#include "ttt_eta.h"
#include "ttt_kernels.h"

namespace ttt {

constexpr int kGenThreads = 256;
constexpr int kGenMaxK = 64;

__host__ __device__ GenLayout::GenLayout(int K_, int F_, int FF_, int NC_, bool mlp_) : K(K_), F(F_), FF(mlp_ ? FF_ : F_), NC(NC_), mlp(mlp_) {
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off += (n + 3) & ~(size_t)3;
    return o;
  };
  state = mlp ? (size_t)F * FF + FF + (size_t)FF * F + F : (size_t)F * F + F;
  state = (state + 3) & ~(size_t)3;
  states = take(state * NC);
  wfin = take(state);
  const size_t KF = (size_t)K * F, KK = (size_t)K * K, KH = (size_t)K * FF;
  xq = take(KF), xk = take(KF), xv = take(KF), dout = take(KF);
  eta = take(KK), a1 = take(KK), c1 = take(KK), a2 = take(KK), c2 = take(KK);
  deta = take(KK), da1 = take(KK), dc1 = take(KK), da2 = take(KK), dc2 = take(KK);
  z1 = take(KH), x2 = take(KH), d1 = take(KH), dd1 = take(KH), p = take(KH), g1 = take(KH);
  z1b = take(KH), x2b = take(KH), db = take(KH);
  z2 = take(KF), z2h = take(KF), g2 = take(KF), z2b = take(KF), z2bh = take(KF);
  sig2 = take(K), sigb = take(K), de = take(K);
  t1 = take(KH), dg1 = take(KH), dx2 = take(KH), dx2b = take(KH), dz1b = take(KH), dp = take(KH), dz1 = take(KH);
  t2 = take(KF), dg2 = take(KF), dz2b = take(KF), dz2 = take(KF), dxq = take(KF), dxk = take(KF), dxv = take(KF);
  lnwt = take(KF), lnbt = take(KF);
  per_chain = off;
}

namespace {

constexpr int kGenStage = 16384;  // floats of LDS staging for one product's operands (64 KB)
// Largest output block (rows or columns) one staged product takes: a chunk
// of 16 contraction steps of both operands, rows padded by 4 floats, must
// fit the staging area, so that every chunk advances the contraction.
constexpr int kGenBlock = 480;
static_assert(kGenStage / ((kGenBlock + 4) + (kGenBlock + 4)) >= 16, "a staged chunk holds 16 contraction steps");

// C[M x N] (row stride ldc) = alpha * op(A) op(B) (+ C when acc), with
// op(A)[i][k] = ta ? A[k * lda + i] : A[i * lda + k] and likewise for B.
// The operands are staged through LDS in chunks of kc contraction steps
// (k-major: As[k][i], Bs[k][j], rows padded by 4 floats; all of a chunk's
// global loads in flight together, read along the operand's contiguous
// dimension), then wave w forms the 16 x 16 output tiles w, w + 4, ... with
// fp32 MFMA (v_mfma_f32_16x16x4_f32: exact products, fp32 sums), its operand
// frags read from LDS (the padding puts the four lane groups of a read on
// distinct banks).  Every thread of the workgroup calls it (it holds
// barriers).  M, N and Kd are multiples of 16, M and N at most kGenBlock.
__device__ void gg_block(float* __restrict__ C, int ldc, const float* __restrict__ A, int lda, bool ta,
                         const float* __restrict__ B, int ldb, bool tb, int M, int N, int Kd, float alpha, bool acc) {
  __shared__ float st[kGenStage];
  const int sa = M + 4, sb = N + 4;  // padded k-row strides: the transposing stores spread over the banks
  const int kc = min(Kd, (kGenStage / (sa + sb)) & ~15);  // >= 16 (kGenBlock)
  float* As = st;
  const int wave = threadIdx.x >> 6, l = lane_id(), g = l >> 4, r = l & 15;
  const int nt = N >> 4, ntile = (M >> 4) * nt;
  for (int k0 = 0; k0 < Kd; k0 += kc) {
    const int kk = min(kc, Kd - k0);
    float* Bs = st + kk * sa;
    if (ta) {  // A[(k0 + k) * lda + i]: i contiguous
#pragma unroll 4
      for (int idx = threadIdx.x; idx < kk * M; idx += kGenThreads) {
        const int k = idx / M, i = idx - k * M;
        As[k * sa + i] = A[(size_t)(k0 + k) * lda + i];
      }
    } else {  // A[i * lda + k0 + k]: k contiguous
#pragma unroll 4
      for (int idx = threadIdx.x; idx < kk * M; idx += kGenThreads) {
        const int i = idx / kk, k = idx - i * kk;
        As[k * sa + i] = A[(size_t)i * lda + k0 + k];
      }
    }
    if (tb) {  // B[j * ldb + k0 + k]: k contiguous
#pragma unroll 4
      for (int idx = threadIdx.x; idx < kk * N; idx += kGenThreads) {
        const int j = idx / kk, k = idx - j * kk;
        Bs[k * sb + j] = B[(size_t)j * ldb + k0 + k];
      }
    } else {  // B[(k0 + k) * ldb + j]: j contiguous
#pragma unroll 4
      for (int idx = threadIdx.x; idx < kk * N; idx += kGenThreads) {
        const int k = idx / N, j = idx - k * N;
        Bs[k * sb + j] = B[(size_t)(k0 + k) * ldb + j];
      }
    }
    __syncthreads();
    for (int t = wave; t < ntile; t += kGenThreads / 64) {
      const int i0 = (t / nt) * 16, j0 = (t - (t / nt) * nt) * 16;
      const float* ap = As + i0 + r;  // lane (g, r): op(A)[i0 + r][k + 4g + j]
      const float* bp = Bs + j0 + r;  //              op(B)[k + 4g + j][j0 + r]
      f4 c = f4{0.f, 0.f, 0.f, 0.f};
      for (int k = 0; k < kk; k += 16) {
        Frag<float> fa, fb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          fa.v[j] = ap[(k + 4 * g + j) * sa];
          fb.v[j] = bp[(k + 4 * g + j) * sb];
        }
        mma16(c, fa, fb);
      }
      // lane (g, r) holds C[i0 + 4g + j][j0 + r]
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float* out = C + (size_t)(i0 + 4 * g + j) * ldc + j0 + r;
        float v = c[j] * alpha;
        if (acc || k0 > 0) v += *out;
        *out = v;
      }
    }
    __syncthreads();  // the staging area is free for the next chunk or product
  }
}

// gg_block over output blocks of at most kGenBlock rows and columns (any M, N
// that are multiples of 16): block (i0, j0) reads rows i0.. of op(A) and
// columns j0.. of op(B) and writes C[i0.., j0..].
__device__ void gg(float* __restrict__ C, int ldc, const float* __restrict__ A, int lda, bool ta,
                   const float* __restrict__ B, int ldb, bool tb, int M, int N, int Kd, float alpha, bool acc) {
  for (int i0 = 0; i0 < M; i0 += kGenBlock) {
    const int mb = min(kGenBlock, M - i0);
    const float* Ab = ta ? A + i0 : A + (size_t)i0 * lda;
    for (int j0 = 0; j0 < N; j0 += kGenBlock) {
      const int nb = min(kGenBlock, N - j0);
      const float* Bb = tb ? B + (size_t)j0 * ldb : B + j0;
      gg_block(C + (size_t)i0 * ldc + j0, ldc, Ab, lda, ta, Bb, ldb, tb, mb, nb, Kd, alpha, acc);
    }
  }
}

__device__ __forceinline__ void copy_f(float* __restrict__ dst, const float* __restrict__ src, size_t n) {
  for (size_t i = threadIdx.x; i < n; i += kGenThreads) dst[i] = src[i];
}

template <typename T> __device__ __forceinline__ float ld(const T* p, size_t i) { return (float)p[i]; }

// state views: W1 [F][FF], b1 [FF], W2 [FF][F], b2 [F] (Linear: W [F][F], b [F])
struct State {
  float *W1, *b1, *W2, *b2;
  __device__ State(float* s, const GenLayout& L) {
    W1 = s;
    b1 = W1 + (size_t)L.F * L.FF;
    W2 = b1 + L.FF;
    b2 = L.mlp ? W2 + (size_t)L.FF * L.F : b1;
  }
};

// the state given as separate tensors of one chain
struct StatePtrs {
  float *W1, *b1, *W2, *b2;
};

__device__ void copy_state_out(const State& s, StatePtrs d, const GenLayout& L, size_t k) {
  const size_t F = L.F, FF = L.FF;
  if (L.mlp) {
    if (d.W1) copy_f(d.W1 + k * F * FF, s.W1, F * FF);
    if (d.b1) copy_f(d.b1 + k * FF, s.b1, FF);
    if (d.W2) copy_f(d.W2 + k * FF * F, s.W2, FF * F);
    if (d.b2) copy_f(d.b2 + k * F, s.b2, F);
  } else {
    if (d.W1) copy_f(d.W1 + k * F * F, s.W1, F * F);
    if (d.b1) copy_f(d.b1 + k * F, s.b1, F);
  }
}

// Row passes over [K x C] blocks: each 16-lane DPP row of the workgroup
// (kRowGroups of them) takes one token row at a time (rows q, q + kRowGroups,
// ...), lane u covering columns u, u + 16, ...; row sums are sum_row16 of the
// lanes' partials.  K is a multiple of 16, so every group makes the same
// number of iterations and all 16 lanes of a DPP row take part in every
// reduction.  Rows held in registers have at most RM columns per lane (the
// kernels are instantiated with RM = 4 for F <= 64 and RM = 16 for F <= 256).
constexpr int kRowGroups = kGenThreads / 16;

__device__ __forceinline__ int row_grp() { return threadIdx.x >> 4; }
__device__ __forceinline__ int row_lane() { return threadIdx.x & 15; }

// Inner-loss LayerNorm fused with the L2 loss's gradient over the K rows of
// Z (the bias added here and written back): normalised rows zh, sigma, and
// G = d loss / d Z (ops/ttt_utils.py:21-48).
template <int RM>
__device__ void ln_l2_rows(float* z, const float* bias, const float* xv, const float* xk, const float* lw,
                           const float* lb, int K, int F, float eps, float* zh, float* sig, float* G) {
  const int u = row_lane(), nf = F >> 4;
  for (int r = row_grp(); r < K; r += kRowGroups) {
    float v[RM], tg[RM];
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < RM; ++q) {
      if (q < nf) {
        const int f = u + 16 * q;
        const size_t i = (size_t)r * F + f;
        v[q] = z[i] + bias[f];
        z[i] = v[q];
        tg[q] = xv[i] - xk[i];
        acc += v[q];
      }
    }
    const float mu = sum_row16(acc) / (float)F;
    acc = 0.f;
#pragma unroll
    for (int q = 0; q < RM; ++q)
      if (q < nf) acc += (v[q] - mu) * (v[q] - mu);
    const float sd = sqrtf(sum_row16(acc) / (float)F + eps);
    float S1 = 0.f, S2 = 0.f;
#pragma unroll
    for (int q = 0; q < RM; ++q) {
      if (q < nf) {
        const int f = u + 16 * q;
        const float xh = (v[q] - mu) / sd;
        const float g = lw[f] * (lw[f] * xh + lb[f] - tg[q]);
        zh[(size_t)r * F + f] = xh;
        v[q] = xh;
        tg[q] = g;
        S1 += g;
        S2 += g * xh;
      }
    }
    S1 = sum_row16(S1);
    S2 = sum_row16(S2);
#pragma unroll
    for (int q = 0; q < RM; ++q)
      if (q < nf) G[(size_t)r * F + u + 16 * q] = ((float)F * tg[q] - S1 - v[q] * S2) / ((float)F * sd);
    if (u == 0) sig[r] = sd;
  }
}

// Column sums over the K rows of a [K x C] block: for every column c < C,
// put(c, t) with t[v] = sum_r val(r, c)[v].  For C < 256 the threads split
// the rows into kGenThreads / C phases whose partials meet in LDS; every
// thread of the workgroup calls it (it holds a barrier).
template <int NV, typename Val, typename Put>
__device__ void col_sums(int K, int C, Val val, Put put) {
  __shared__ float red[NV][kGenThreads];
  if (C >= kGenThreads) {
    for (int c = threadIdx.x; c < C; c += kGenThreads) {
      float t[NV] = {};
#pragma unroll 8
      for (int r = 0; r < K; ++r) val(r, c, t);
      put(c, t);
    }
    return;
  }
  const int P = kGenThreads / C;  // row phases
  const int c = threadIdx.x % C, ph = threadIdx.x / C;
  float t[NV] = {};
  if (ph < P) {
#pragma unroll 4
    for (int r = ph; r < K; r += P) val(r, c, t);
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) red[v][threadIdx.x] = t[v];
  __syncthreads();
  if (threadIdx.x < C) {
    float tot[NV] = {};
    for (int q = 0; q < P; ++q)
#pragma unroll
      for (int v = 0; v < NV; ++v) tot[v] += red[v][q * C + threadIdx.x];
    put(threadIdx.x, tot);
  }
  __syncthreads();  // red is free for the next call
}

struct GenArgs {
  const void *XQ, *XK, *XV, *eta, *dout;
  const float *ln_w, *ln_b;
  const float *W1_init, *b1_init, *W2_init, *b2_init;
  void* out;
  StatePtrs last, ckpt, memo;
  void *dXQ, *dXK, *dXV, *deta;
  float *dW1, *db1, *dW2, *db2, *dln_w, *dln_b;
  float* saved;
  int B, H, NC, K, F, FF, G, M, eta_rule;
  bool mlp;
  float eps;
};

// Forward values of mini-batch s from state S into the chain's scratch; with
// `emit`, also its output rows and the state after it (into `next`).
template <typename T, int RM>
__device__ void gen_step_fwd(const GenArgs& a, const GenLayout& L, float* sc, size_t chain, int s, const State& S,
                             bool emit, const State* next) {
  const int K = L.K, F = L.F, FF = L.FF;
  const int h = (int)(chain % a.H);
  const float* lw = a.ln_w + (size_t)h * F;
  const float* lb = a.ln_b + (size_t)h * F;
  const size_t row0 = (chain * a.NC + s) * K;  // first token row of the mini-batch
  float *xq = sc + L.xq, *xk = sc + L.xk, *xv = sc + L.xv, *eta = sc + L.eta;
  const T *XQ = static_cast<const T*>(a.XQ), *XK = static_cast<const T*>(a.XK), *XV = static_cast<const T*>(a.XV);
  #pragma unroll 4
  for (size_t i = threadIdx.x; i < (size_t)K * F; i += kGenThreads) {
    xq[i] = ld(XQ, row0 * F + i);
    xk[i] = ld(XK, row0 * F + i);
    xv[i] = ld(XV, row0 * F + i);
  }
  #pragma unroll 4
  for (int i = threadIdx.x; i < K * K; i += kGenThreads) {
    const int r = i / K, c = i % K;
    if (a.eta_rule == TTT_ETA_DENSE) {
      eta[i] = ld(static_cast<const T*>(a.eta), (chain * a.NC + s) * K * K + i);
    } else if (a.eta_rule == TTT_ETA_DENSE_F32) {
      eta[i] = static_cast<const float*>(a.eta)[(chain * a.NC + s) * K * K + i];
    } else {
      const float lr = static_cast<const float*>(a.eta)[row0 + c];
      eta[i] = a.eta_rule == TTT_ETA_LAYER ? lr * (1.0f / (float)K) : (c <= r ? lr * (1.0f / (float)(r + 1)) : 0.0f);
    }
  }
  __syncthreads();
  float *a1 = sc + L.a1, *c1 = sc + L.c1, *g2 = sc + L.g2, *z2 = sc + L.z2, *z2h = sc + L.z2h, *sig2 = sc + L.sig2;
  float *z2b = sc + L.z2b, *z2bh = sc + L.z2bh, *sigb = sc + L.sigb;
  gg(a1, K, xq, F, false, xk, F, true, K, K, F, 1.f, false);
  if (L.mlp) {
    float *z1 = sc + L.z1, *x2 = sc + L.x2, *d1 = sc + L.d1, *dd1 = sc + L.dd1, *p = sc + L.p, *g1 = sc + L.g1;
    float *z1b = sc + L.z1b, *x2b = sc + L.x2b, *db = sc + L.db, *a2 = sc + L.a2, *c2 = sc + L.c2;
    gg(z1, FF, xk, F, false, S.W1, FF, false, K, FF, F, 1.f, false);
    __syncthreads();
    #pragma unroll 4
    for (int i = threadIdx.x; i < K * FF; i += kGenThreads) {
      float y, dy, ddy;
      gelu_all(z1[i] + S.b1[i % FF], y, dy, ddy);
      x2[i] = y;
      d1[i] = dy;
      dd1[i] = ddy;
    }
    #pragma unroll 4
    for (int i = threadIdx.x; i < K * K; i += kGenThreads) c1[i] = eta[i] * (a1[i] + 1.0f);
    __syncthreads();
    gg(z2, F, x2, FF, false, S.W2, F, false, K, F, FF, 1.f, false);
    __syncthreads();
    ln_l2_rows<RM>(z2, S.b2, xv, xk, lw, lb, K, F, a.eps, z2h, sig2, g2);
    __syncthreads();
    gg(p, FF, g2, F, false, S.W2, F, true, K, FF, F, 1.f, false);
    __syncthreads();
    #pragma unroll 4
    for (int i = threadIdx.x; i < K * FF; i += kGenThreads) g1[i] = p[i] * d1[i];
    __syncthreads();
    gg(z1b, FF, xq, F, false, S.W1, FF, false, K, FF, F, 1.f, false);
    gg(z1b, FF, c1, K, false, g1, FF, false, K, FF, K, -1.f, true);
    __syncthreads();
    #pragma unroll 4
    for (int i = threadIdx.x; i < K * FF; i += kGenThreads) {
      float y, dy, ddy;
      gelu_all(z1b[i] + S.b1[i % FF], y, dy, ddy);
      x2b[i] = y;
      db[i] = dy;
    }
    __syncthreads();
    gg(a2, K, x2b, FF, false, x2, FF, true, K, K, FF, 1.f, false);
    __syncthreads();
    #pragma unroll 4
    for (int i = threadIdx.x; i < K * K; i += kGenThreads) c2[i] = eta[i] * (a2[i] + 1.0f);
    __syncthreads();
    gg(z2b, F, x2b, FF, false, S.W2, F, false, K, F, FF, 1.f, false);
    gg(z2b, F, c2, K, false, g2, F, false, K, F, K, -1.f, true);
  } else {
    gg(z2, F, xk, F, false, S.W1, F, false, K, F, F, 1.f, false);
    __syncthreads();
    #pragma unroll 4
    for (int i = threadIdx.x; i < K * K; i += kGenThreads) c1[i] = eta[i] * (a1[i] + 1.0f);
    ln_l2_rows<RM>(z2, S.b1, xv, xk, lw, lb, K, F, a.eps, z2h, sig2, g2);
    __syncthreads();
    gg(z2b, F, xq, F, false, S.W1, F, false, K, F, F, 1.f, false);
    gg(z2b, F, c1, K, false, g2, F, false, K, F, K, -1.f, true);
  }
  __syncthreads();
  // output LayerNorm and residual
  const float* bo = L.mlp ? S.b2 : S.b1;
  {
    const int u = row_lane(), nf = F >> 4;
    for (int r = row_grp(); r < K; r += kRowGroups) {
      float v[RM];
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < RM; ++q) {
        if (q < nf) {
          const size_t i = (size_t)r * F + u + 16 * q;
          v[q] = z2b[i] + bo[u + 16 * q];
          z2b[i] = v[q];
          acc += v[q];
        }
      }
      const float mu = sum_row16(acc) / (float)F;
      acc = 0.f;
#pragma unroll
      for (int q = 0; q < RM; ++q)
        if (q < nf) acc += (v[q] - mu) * (v[q] - mu);
      const float sd = sqrtf(sum_row16(acc) / (float)F + a.eps);
      if (u == 0) sigb[r] = sd;
#pragma unroll
      for (int q = 0; q < RM; ++q) {
        if (q < nf) {
          const int f = u + 16 * q;
          const size_t i = (size_t)r * F + f;
          const float xh = (v[q] - mu) / sd;
          z2bh[i] = xh;
          if (emit) static_cast<T*>(a.out)[(row0 + r) * F + f] = (T)(xq[i] + lw[f] * xh + lb[f]);
        }
      }
    }
  }
  if (!emit) return;
  // state after the mini-batch: W -= X^T diag(e) G, b -= G^T e with e = eta[K-1]
  float* u1 = sc + L.t1;  // e-scaled G1 (MLP)
  float* u2 = sc + L.t2;  // e-scaled G2 / G
  const float* e = eta + (size_t)(K - 1) * K;
  #pragma unroll 4
  for (int i = threadIdx.x; i < K * F; i += kGenThreads) u2[i] = e[i / F] * g2[i];
  if (L.mlp)
    #pragma unroll 4
    for (int i = threadIdx.x; i < K * FF; i += kGenThreads) u1[i] = e[i / FF] * sc[L.g1 + i];
  copy_f(next->W1, S.W1, L.state);  // the whole state block
  __syncthreads();
  if (L.mlp) {
    gg(next->W1, FF, xk, F, true, u1, FF, false, F, FF, K, -1.f, true);
    gg(next->W2, F, sc + L.x2, FF, true, u2, F, false, FF, F, K, -1.f, true);
    col_sums<1>(K, FF, [&](int r, int c, float(&t)[1]) { t[0] += u1[(size_t)r * FF + c]; },
                [&](int c, const float(&t)[1]) { next->b1[c] -= t[0]; });
    col_sums<1>(K, F, [&](int r, int c, float(&t)[1]) { t[0] += u2[(size_t)r * F + c]; },
                [&](int c, const float(&t)[1]) { next->b2[c] -= t[0]; });
  } else {
    gg(next->W1, F, xk, F, true, u2, F, false, F, F, K, -1.f, true);
    col_sums<1>(K, F, [&](int r, int c, float(&t)[1]) { t[0] += u2[(size_t)r * F + c]; },
                [&](int c, const float(&t)[1]) { next->b1[c] -= t[0]; });
  }
  __syncthreads();
}

template <typename T, int RM>
__global__ __launch_bounds__(kGenThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void gen_fwd_kernel(GenArgs a) {
  const size_t chain = blockIdx.x;
  const GenLayout L(a.K, a.F, a.FF, a.NC, a.mlp);
  float* base = a.saved + chain * L.per_chain;
  auto state_at = [&](int s) { return State(base + L.states + (size_t)s * L.state, L); };
  {
    const State s0 = state_at(0);
    const size_t F = L.F, FF = L.FF;
    copy_f(s0.W1, a.W1_init + chain * F * FF, F * FF);
    copy_f(s0.b1, a.b1_init + chain * FF, FF);
    if (L.mlp) {
      copy_f(s0.W2, a.W2_init + chain * FF * F, FF * F);
      copy_f(s0.b2, a.b2_init + chain * F, F);
    }
  }
  __syncthreads();
  auto off = [&](StatePtrs p, size_t k0) {  // the chain's block of a [B,H,n,...] state tensor set
    StatePtrs q = p;
    const size_t F = L.F, FF = L.FF;
    if (q.W1) q.W1 += k0 * F * FF;
    if (q.b1) q.b1 += k0 * FF;
    if (q.W2) q.W2 += k0 * FF * F;
    if (q.b2) q.b2 += k0 * F;
    return q;
  };
  const int NK = (a.NC + a.G - 1) / a.G, NS = (a.NC + a.M - 1) / a.M;
  const StatePtrs ck = off(a.ckpt, chain * NK), mm = off(a.memo, chain * NS), la = off(a.last, chain);
  for (int s = 0; s < a.NC; ++s) {
    const State S = state_at(s);
    if (s % a.G == 0) copy_state_out(S, ck, L, s / a.G);
    const State nxt = s + 1 < a.NC ? state_at(s + 1) : State(base + L.wfin, L);
    gen_step_fwd<T, RM>(a, L, base, chain, s, S, true, &nxt);
    if (a.memo.W1 && s % a.M == 0) copy_state_out(nxt, mm, L, s / a.M);
    if (s + 1 == a.NC && a.last.W1) copy_state_out(nxt, la, L, 0);
    __syncthreads();
  }
}

template <typename T, int RM>
__global__ __launch_bounds__(kGenThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void gen_bwd_kernel(GenArgs a) {
  const size_t chain = blockIdx.x;
  const GenLayout L(a.K, a.F, a.FF, a.NC, a.mlp);
  const int K = L.K, F = L.F, FF = L.FF;
  const int h = (int)(chain % a.H);
  const float* lw = a.ln_w + (size_t)h * F;
  const float* lb = a.ln_b + (size_t)h * F;
  float* sc = a.saved + chain * L.per_chain;
  // gradient wrt the running state: starts at zero (the final state's gradient)
  float* dW1 = a.dW1 + chain * (size_t)F * FF;
  float* db1 = a.db1 + chain * (size_t)FF;
  float* dW2 = L.mlp ? a.dW2 + chain * (size_t)FF * F : nullptr;
  float* db2 = L.mlp ? a.db2 + chain * (size_t)F : nullptr;
  float* dlnw = a.dln_w + chain * (size_t)F;
  float* dlnb = a.dln_b + chain * (size_t)F;
  for (int i = threadIdx.x; i < F * FF; i += kGenThreads) dW1[i] = 0.f;
  for (int i = threadIdx.x; i < FF; i += kGenThreads) db1[i] = 0.f;
  if (L.mlp) {
    for (int i = threadIdx.x; i < FF * F; i += kGenThreads) dW2[i] = 0.f;
    for (int i = threadIdx.x; i < F; i += kGenThreads) db2[i] = 0.f;
  }
  for (int i = threadIdx.x; i < F; i += kGenThreads) {
    dlnw[i] = 0.f;
    dlnb[i] = 0.f;
  }
  float *xq = sc + L.xq, *xk = sc + L.xk, *xv = sc + L.xv, *eta = sc + L.eta, *dout = sc + L.dout;
  float *a1 = sc + L.a1, *c1 = sc + L.c1, *deta = sc + L.deta, *da1 = sc + L.da1, *dc1 = sc + L.dc1;
  float *g2 = sc + L.g2, *z2h = sc + L.z2h, *sig2 = sc + L.sig2, *z2bh = sc + L.z2bh, *sigb = sc + L.sigb;
  float *t2 = sc + L.t2, *dg2 = sc + L.dg2, *dz2b = sc + L.dz2b, *dz2 = sc + L.dz2;
  float *dxq = sc + L.dxq, *dxk = sc + L.dxk, *dxv = sc + L.dxv, *de = sc + L.de, *lnwt = sc + L.lnwt,
        *lnbt = sc + L.lnbt;
  float *x2 = sc + L.x2, *d1 = sc + L.d1, *dd1 = sc + L.dd1, *p = sc + L.p, *g1 = sc + L.g1, *x2b = sc + L.x2b,
        *dbv = sc + L.db, *a2 = sc + L.a2, *c2 = sc + L.c2, *da2 = sc + L.da2, *dc2 = sc + L.dc2;
  float *t1 = sc + L.t1, *dg1 = sc + L.dg1, *dx2 = sc + L.dx2, *dx2b = sc + L.dx2b, *dz1b = sc + L.dz1b,
        *dp = sc + L.dp, *dz1 = sc + L.dz1;
  __syncthreads();
  for (int s = a.NC - 1; s >= 0; --s) {
    const State S(sc + L.states + (size_t)s * L.state, L);
    gen_step_fwd<T, RM>(a, L, sc, chain, s, S, false, nullptr);
    const size_t row0 = (chain * a.NC + s) * K;
    #pragma unroll 4
    for (size_t i = threadIdx.x; i < (size_t)K * F; i += kGenThreads)
      dout[i] = ld(static_cast<const T*>(a.dout), row0 * F + i);
    __syncthreads();
    const float* e = eta + (size_t)(K - 1) * K;
    // ---- through the state update W' = W - X^T diag(e) G, b' = b - G^T e
    // (the running state gradient is dL/dW' here)
    if (L.mlp) {
      gg(t1, FF, xk, F, false, dW1, FF, false, K, FF, F, 1.f, false);  // XK dW1'
      gg(t2, F, x2, FF, false, dW2, F, false, K, F, FF, 1.f, false);   // X2 dW2'
      gg(dx2, FF, g2, F, false, dW2, F, true, K, FF, F, 1.f, false);   // G2 dW2'^T
      gg(dxk, F, g1, FF, false, dW1, FF, true, K, F, FF, 1.f, false);  // G1 dW1'^T
    } else {
      gg(t2, F, xk, F, false, dW1, F, false, K, F, F, 1.f, false);   // XK dW'
      gg(dxk, F, g2, F, false, dW1, F, true, K, F, F, 1.f, false);   // G dW'^T
    }
    __syncthreads();
    {
      const int u = row_lane(), nf = F >> 4;
      for (int r = row_grp(); r < K; r += kRowGroups) {
        const float er = e[r];
        float d = 0.f;
        if (L.mlp) {
#pragma unroll 4
          for (int c = u; c < FF; c += 16) {
            const size_t i = (size_t)r * FF + c;
            const float t = t1[i] + db1[c];
            d -= t * g1[i];
            dg1[i] = -er * t;
            dx2[i] *= -er;
          }
#pragma unroll 4
          for (int c = u; c < F; c += 16) {
            const size_t i = (size_t)r * F + c;
            const float t = t2[i] + db2[c];
            d -= t * g2[i];
            dg2[i] = -er * t;
            dxk[i] *= -er;
          }
        } else {
#pragma unroll 4
          for (int c = u; c < F; c += 16) {
            const size_t i = (size_t)r * F + c;
            const float t = t2[i] + db1[c];
            d -= t * g2[i];
            dg2[i] = -er * t;
            dxk[i] *= -er;
          }
        }
        d = sum_row16(d);
        if (u == 0) de[r] = d;
        // ---- output LayerNorm: out = XQ + ln_w * zbh + ln_b
        const float sd = sigb[r];
        float dh[RM], zh[RM];
        float m1 = 0.f, m2 = 0.f;
#pragma unroll
        for (int q = 0; q < RM; ++q) {
          if (q < nf) {
            const int f = u + 16 * q;
            const size_t i = (size_t)r * F + f;
            dh[q] = dout[i] * lw[f];
            zh[q] = z2bh[i];
            m1 += dh[q];
            m2 += dh[q] * zh[q];
          }
        }
        m1 = sum_row16(m1) / (float)F;
        m2 = sum_row16(m2) / (float)F;
#pragma unroll
        for (int q = 0; q < RM; ++q) {
          if (q < nf) {
            const size_t i = (size_t)r * F + u + 16 * q;
            dz2b[i] = (dh[q] - m1 - zh[q] * m2) / sd;
            dxq[i] = dout[i];
          }
        }
      }
    }
    __syncthreads();
    float* dbo = L.mlp ? db2 : db1;
    col_sums<3>(
        K, F,
        [&](int r, int f, float(&t)[3]) {
          const size_t i = (size_t)r * F + f;
          t[0] += dout[i] * z2bh[i];
          t[1] += dout[i];
          t[2] += dz2b[i];
        },
        [&](int f, const float(&t)[3]) {
          dlnw[f] += t[0];
          dlnb[f] += t[1];
          dbo[f] += t[2];
        });
    if (L.mlp) {
      // ---- Z2b = X2b W2 + b2 - (eta o (X2b X2^T + 1)) G2
      gg(dW2, F, x2b, FF, true, dz2b, F, false, FF, F, K, 1.f, true);
      gg(dx2b, FF, dz2b, F, false, S.W2, F, true, K, FF, F, 1.f, false);
      gg(dc2, K, dz2b, F, false, g2, F, true, K, K, F, -1.f, false);
      __syncthreads();
      gg(dg2, F, c2, K, true, dz2b, F, false, K, F, K, -1.f, true);
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * K; i += kGenThreads) {
        deta[i] = dc2[i] * (a2[i] + 1.0f);
        da2[i] = dc2[i] * eta[i];
      }
      __syncthreads();
      gg(dx2b, FF, da2, K, false, x2, FF, false, K, FF, K, 1.f, true);
      gg(dx2, FF, da2, K, true, x2b, FF, false, K, FF, K, 1.f, true);
      __syncthreads();
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * FF; i += kGenThreads) dz1b[i] = dx2b[i] * dbv[i];
      __syncthreads();
      // ---- Z1b = XQ W1 + b1 - (eta o (XQ XK^T + 1)) G1
      col_sums<1>(K, FF, [&](int r, int c, float(&t)[1]) { t[0] += dz1b[(size_t)r * FF + c]; },
                  [&](int c, const float(&t)[1]) { db1[c] += t[0]; });
      gg(dxq, F, dz1b, FF, false, S.W1, FF, true, K, F, FF, 1.f, true);
      gg(dW1, FF, xq, F, true, dz1b, FF, false, F, FF, K, 1.f, true);
      gg(dc1, K, dz1b, FF, false, g1, FF, true, K, K, FF, -1.f, false);
      __syncthreads();
      gg(dg1, FF, c1, K, true, dz1b, FF, false, K, FF, K, -1.f, true);
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * K; i += kGenThreads) {
        deta[i] += dc1[i] * (a1[i] + 1.0f);
        da1[i] = dc1[i] * eta[i];
      }
      __syncthreads();
      gg(dxq, F, da1, K, false, xk, F, false, K, F, K, 1.f, true);
      gg(dxk, F, da1, K, true, xq, F, false, K, F, K, 1.f, true);
      // ---- G1 = (G2 W2^T) o gelu'(Z1)
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * FF; i += kGenThreads) {
        dp[i] = dg1[i] * d1[i];
        dz1[i] = dg1[i] * p[i] * dd1[i];
      }
      __syncthreads();
      gg(dg2, F, dp, FF, false, S.W2, F, false, K, F, FF, 1.f, true);
      gg(dW2, F, dp, FF, true, g2, F, false, FF, F, K, 1.f, true);
      __syncthreads();
    } else {
      // ---- Zb = XQ W + b - (eta o (XQ XK^T + 1)) G
      gg(dW1, F, xq, F, true, dz2b, F, false, F, F, K, 1.f, true);
      gg(dxq, F, dz2b, F, false, S.W1, F, true, K, F, F, 1.f, true);
      gg(dc1, K, dz2b, F, false, g2, F, true, K, K, F, -1.f, false);
      __syncthreads();
      gg(dg2, F, c1, K, true, dz2b, F, false, K, F, K, -1.f, true);
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * K; i += kGenThreads) {
        deta[i] = dc1[i] * (a1[i] + 1.0f);
        da1[i] = dc1[i] * eta[i];
      }
      __syncthreads();
      gg(dxq, F, da1, K, false, xk, F, false, K, F, K, 1.f, true);
      gg(dxk, F, da1, K, true, xq, F, false, K, F, K, 1.f, true);
      __syncthreads();
    }
    // ---- G = LN-fused-L2 gradient of Z (Z2 for the MLP): its backward
    {
      const int u = row_lane(), nf = F >> 4;
      for (int r = row_grp(); r < K; r += kRowGroups) {
        const float sd = sig2[r];
        float xh[RM], qv[RM], rr[RM];
        float S2 = 0.f, Q1 = 0.f, Q2 = 0.f, QG = 0.f;
#pragma unroll
        for (int q = 0; q < RM; ++q) {
          if (q < nf) {
            const int f = u + 16 * q;
            const size_t i = (size_t)r * F + f;
            xh[q] = z2h[i];
            qv[q] = dg2[i];
            rr[q] = lw[f] * xh[q] + lb[f] - (xv[i] - xk[i]);
            const float g = lw[f] * rr[q];
            S2 += g * xh[q];
            Q1 += qv[q];
            Q2 += qv[q] * xh[q];
            QG += qv[q] * g2[i];
          }
        }
        S2 = sum_row16(S2);
        Q1 = sum_row16(Q1);
        Q2 = sum_row16(Q2);
        QG = sum_row16(QG);
        const float inv = 1.0f / ((float)F * sd);
        const float dsig = -QG / sd;
        float m1 = 0.f, m2 = 0.f;
        // pass 1: dg, dt, the LN-parameter terms and dxh (kept in qv)
#pragma unroll
        for (int q = 0; q < RM; ++q) {
          if (q < nf) {
            const int f = u + 16 * q;
            const size_t i = (size_t)r * F + f;
            const float g = lw[f] * rr[q];
            const float dg = ((float)F * qv[q] - Q1 - xh[q] * Q2) * inv;
            const float dxh = (-qv[q] * S2 - g * Q2) * inv + dg * lw[f] * lw[f];
            const float dt = -dg * lw[f];
            dxv[i] = dt;
            dxk[i] -= dt;
            lnwt[i] = dg * (rr[q] + lw[f] * xh[q]);
            lnbt[i] = dg * lw[f];
            qv[q] = dxh;
            m1 += dxh;
            m2 += dxh * xh[q];
          }
        }
        m1 = sum_row16(m1) / (float)F;
        m2 = sum_row16(m2) / (float)F;
#pragma unroll
        for (int q = 0; q < RM; ++q)
          if (q < nf)
            dz2[(size_t)r * F + u + 16 * q] = (qv[q] - m1 - xh[q] * m2) / sd + dsig * xh[q] / (float)F;
      }
    }
    __syncthreads();
    col_sums<3>(
        K, F,
        [&](int r, int f, float(&t)[3]) {
          const size_t i = (size_t)r * F + f;
          t[0] += lnwt[i];
          t[1] += lnbt[i];
          t[2] += dz2[i];
        },
        [&](int f, const float(&t)[3]) {
          dlnw[f] += t[0];
          dlnb[f] += t[1];
          dbo[f] += t[2];
        });
    if (L.mlp) {
      // ---- Z2 = X2 W2 + b2, X2 = gelu(Z1), Z1 = XK W1 + b1
      gg(dx2, FF, dz2, F, false, S.W2, F, true, K, FF, F, 1.f, true);
      gg(dW2, F, x2, FF, true, dz2, F, false, FF, F, K, 1.f, true);
      __syncthreads();
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * FF; i += kGenThreads) dz1[i] += dx2[i] * d1[i];
      __syncthreads();
      col_sums<1>(K, FF, [&](int r, int c, float(&t)[1]) { t[0] += dz1[(size_t)r * FF + c]; },
                  [&](int c, const float(&t)[1]) { db1[c] += t[0]; });
      gg(dxk, F, dz1, FF, false, S.W1, FF, true, K, F, FF, 1.f, true);
      gg(dW1, FF, xk, F, true, dz1, FF, false, F, FF, K, 1.f, true);
    } else {
      // ---- Z = XK W + b
      gg(dxk, F, dz2, F, false, S.W1, F, true, K, F, F, 1.f, true);
      gg(dW1, F, xk, F, true, dz2, F, false, F, F, K, 1.f, true);
    }
    __syncthreads();
    for (int j = threadIdx.x; j < K; j += kGenThreads) deta[(size_t)(K - 1) * K + j] += de[j];
    __syncthreads();
    // ---- this mini-batch's input gradients
    T *DXQ = static_cast<T*>(a.dXQ), *DXK = static_cast<T*>(a.dXK), *DXV = static_cast<T*>(a.dXV);
    #pragma unroll 4
    for (size_t i = threadIdx.x; i < (size_t)K * F; i += kGenThreads) {
      DXQ[row0 * F + i] = (T)dxq[i];
      DXK[row0 * F + i] = (T)dxk[i];
      DXV[row0 * F + i] = (T)dxv[i];
    }
    if (a.eta_rule == TTT_ETA_DENSE) {
      T* DE = static_cast<T*>(a.deta) + (chain * a.NC + s) * K * K;
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * K; i += kGenThreads) DE[i] = (T)deta[i];
    } else if (a.eta_rule == TTT_ETA_DENSE_F32) {
      float* DE = static_cast<float*>(a.deta) + (chain * a.NC + s) * K * K;
      #pragma unroll 4
      for (int i = threadIdx.x; i < K * K; i += kGenThreads) DE[i] = deta[i];
    } else {
      float* DL = static_cast<float*>(a.deta) + row0;
      const bool layer = a.eta_rule == TTT_ETA_LAYER;
      col_sums<1>(
          K, K,
          [&](int i, int j, float(&t)[1]) {
            const float coef = layer ? 1.0f / (float)K : (j <= i ? 1.0f / (float)(i + 1) : 0.f);
            t[0] += deta[(size_t)i * K + j] * coef;
          },
          [&](int j, const float(&t)[1]) { DL[j] = t[0]; });
    }
    __syncthreads();
  }
}

template <typename T, int RM> hipError_t launch_gen_rm(const GenArgs& a, bool bwd, hipStream_t stream) {
  if (bwd)
    hipLaunchKernelGGL((gen_bwd_kernel<T, RM>), dim3(a.B * a.H), dim3(kGenThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((gen_fwd_kernel<T, RM>), dim3(a.B * a.H), dim3(kGenThreads), 0, stream, a);
  return hipGetLastError();
}
template <typename T> hipError_t launch_gen(const GenArgs& a, bool bwd, hipStream_t stream) {
  return a.F <= 64 ? launch_gen_rm<T, 4>(a, bwd, stream) : launch_gen_rm<T, 16>(a, bwd, stream);
}

}  // namespace

bool gen_shape_ok(int K, int F, int FF, bool mlp) {
  if (K < 16 || K > kGenMaxK || K % 16) return false;
  if (F < 16 || F > 256 || F % 16) return false;
  if (mlp && (FF < 16 || FF > 1024 || FF % 16)) return false;
  return true;
}

size_t gen_saved_bytes(int B, int H, int NC, int K, int F, int FF, bool mlp) {
  return (size_t)B * H * GenLayout(K, F, FF, NC, mlp).per_chain * sizeof(float);
}

hipError_t launch_gen_fwd(const GenFwdParams& q, int dtype, hipStream_t stream) {
  if (small_shape_ok(q.K, q.F, q.FF, q.mlp) && !gen_force_general()) return launch_small_fwd(q, dtype, stream);
  GenArgs a{};
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
  a.last = StatePtrs{q.W1_last, q.b1_last, q.W2_last, q.b2_last};
  a.ckpt = StatePtrs{q.W1_ckpt, q.b1_ckpt, q.W2_ckpt, q.b2_ckpt};
  a.memo = StatePtrs{q.W1_memo, q.b1_memo, q.W2_memo, q.b2_memo};
  a.saved = static_cast<float*>(q.saved);
  a.B = q.B;
  a.H = q.H;
  a.NC = q.NC;
  a.K = q.K;
  a.F = q.F;
  a.FF = q.mlp ? q.FF : q.F;
  a.G = q.G;
  a.M = q.M;
  a.eta_rule = q.eta_rule;
  a.mlp = q.mlp;
  a.eps = q.eps;
  if (dtype == TTT_DTYPE_BF16) return launch_gen<__bf16>(a, false, stream);
  if (dtype == TTT_DTYPE_F16) return launch_gen<_Float16>(a, false, stream);
  return launch_gen<float>(a, false, stream);
}

hipError_t launch_gen_bwd(const GenBwdParams& q, int dtype, hipStream_t stream) {
  if (small_shape_ok(q.K, q.F, q.FF, q.mlp) && !gen_force_general()) return launch_small_bwd(q, dtype, stream);
  GenArgs a{};
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
  a.saved = static_cast<float*>(q.saved);
  a.B = q.B;
  a.H = q.H;
  a.NC = q.NC;
  a.K = q.K;
  a.F = q.F;
  a.FF = q.mlp ? q.FF : q.F;
  a.G = 1;
  a.M = 1;
  a.eta_rule = q.eta_rule;
  a.mlp = q.mlp;
  a.eps = q.eps;
  if (dtype == TTT_DTYPE_BF16) return launch_gen<__bf16>(a, true, stream);
  if (dtype == TTT_DTYPE_F16) return launch_gen<_Float16>(a, true, stream);
  return launch_gen<float>(a, true, stream);
}

}  // namespace ttt
