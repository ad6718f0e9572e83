// TTT-MLP memory-cache combiner on gfx950 (ttt_layer.py:506-561).
//
// The sequence is cut into segments of M mini-batches; memo state j is the
// fast weight the forward snapshot after mini-batch j*M.  For a token t of
// segment i >= 1, with summary_j = mean of XK over segment j and
// gamma = softmax_j(XU_t . summary_j) over j = 0..i,
//
//   out_t = gamma_i XQW_t + sum_{j<i} gamma_j R_j(XQ_t),
//   R_j(x) = x + LN_eps(gelu(x W1_j + b1_j) W2_j + b2_j) * ln_w + ln_b,
//
// and segment 0 keeps XQW.  The reference runs this as a Python loop with one
// cached-readout launch per (segment, memo state) pair; here it is three
// launches forward and two backward:
//
//   memo_summary_kernel   one workgroup per (chain, segment): the segment summaries;
//   memo_gate_kernel      one thread per token: the gates (written as
//                         gamma^T [NS][tokens] plus the current-segment gate);
//   memo_combine_kernel   one workgroup per (chain, pair of 256-token chunks):
//                         for each memo state j below a chunk's last segment, stage
//                         W1_j/W2_j into LDS in MFMA operand order (as the cached
//                         readout does), run the chunk's tiles of later
//                         segments through R_j and accumulate gamma_j R_j (forward)
//                         or dOut . R_j (backward: the gate gradients);
//   memo_finish_kernel    (backward) one thread per token: the softmax
//                         backward, dXU = sum_j dsims_j summary_j and
//                         dXQW = gamma_i dOut;
//   memo_dxk_kernel       (backward) one workgroup per (chain, segment):
//                         dXK = mean over the segment's tokens of
//                         dsims_current XU, the same for each of its tokens.
//
// Gradients flow into XQW, XU and XK.  The cached readouts carry none, and a
// segment's summary carries one only as the current summary of its own
// tokens' gates (the reference caches it detached).  The gates buffer per
// chain (fp32) holds gamma^T [NS][NT], the current gate [NT], the summaries
// [NS][F] and, in the backward, the gate gradients [NS][NT] and the
// current-summary logit gradients [NT] (NT = NC * 16 tokens).
#include "ttt_kernels.h"

namespace ttt {

constexpr int kMemoThreads = 256;

struct MemoGateLayout {
  size_t gam, gcur, summ, dgam, dscur, stride;  // float offsets within a chain's block
  __host__ __device__ MemoGateLayout(int NC, int K, int F, int NS) {
    const size_t NT = (size_t)NC * K;
    gam = 0;
    gcur = gam + (size_t)NS * NT;
    summ = gcur + NT;
    dgam = summ + (size_t)NS * F;
    dscur = dgam + (size_t)NS * NT;
    stride = (dscur + NT + 3) & ~(size_t)3;
  }
};

size_t memo_gate_floats_per_chain(int NC, int K, int F, int M) {
  const int NS = (NC + M - 1) / M;
  return MemoGateLayout(NC, K, F, NS).stride;
}

// ------------------------------------------------------------------ summaries and gates
constexpr int kSegThreads = 256;  // threads of the per-(chain, segment) kernels

// Sum over a segment's tokens t0..t1-1 of w(t) * X[t][f], for f = threadIdx.x % F,
// kSegThreads / F token rows at a time; the block's total for column f is returned
// to every thread of that column.
template <typename T, int F, typename W>
__device__ __forceinline__ float segment_column_sum(const T* __restrict__ X, int t0, int t1, W w, float* part) {
  constexpr int R = kSegThreads / F;
  const int f = threadIdx.x % F, r = threadIdx.x / F;
  float acc = 0.f;
#pragma unroll 4
  for (int t = t0 + r; t < t1; t += R) acc += w(t) * (float)X[(size_t)t * F + f];
  part[threadIdx.x] = acc;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int q = 0; q < R; ++q) tot += part[q * F + f];
  return tot;
}

// one workgroup per (chain, segment): mean of XK over the segment
template <typename T, int F>
__global__ __launch_bounds__(kSegThreads) void memo_summary_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  __shared__ float part[kSegThreads];
  const int chain = blockIdx.x / p.NS, j = blockIdx.x - chain * p.NS;
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const MemoGateLayout L(NC, K, F, NS);
  const T* __restrict__ XK = static_cast<const T*>(p.XK) + (size_t)chain * NT * F;
  const int t0 = j * M * K, t1 = min((j + 1) * M, NC) * K;
  const float tot = segment_column_sum<T, F>(XK, t0, t1, [](int) { return 1.0f; }, part);
  if (threadIdx.x < F) p.gates[(size_t)chain * L.stride + L.summ + (size_t)j * F + threadIdx.x] = tot / (float)(t1 - t0);
}

// one workgroup per (chain, block of kMemoThreads tokens), one token per thread:
// the softmax over the summaries of segments 0..i
template <typename T, int F>
__global__ __launch_bounds__(kMemoThreads) void memo_gate_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  const int nblk = (p.NC * K + kMemoThreads - 1) / kMemoThreads;
  const int chain = blockIdx.x / nblk, blk = blockIdx.x - chain * nblk;
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const MemoGateLayout L(NC, K, F, NS);
  float* __restrict__ gb = p.gates + (size_t)chain * L.stride;
  __shared__ f4 summ[kMemoMaxStates * F / 4];
  const int t = blk * kMemoThreads + threadIdx.x;
  const int tmax = min(NT, (blk + 1) * kMemoThreads) - 1;
  const int ns = (tmax / K) / M + 1;  // segments this block's tokens can reach
  for (int q = threadIdx.x; q < ns * F / 4; q += kMemoThreads)
    summ[q] = *reinterpret_cast<const f4*>(gb + L.summ + 4 * (size_t)q);
  __syncthreads();
  if (t >= NT) return;  // (no barrier follows)
  const int i = (t / K) / M;
  if (i == 0) {
    gb[L.gcur + t] = 1.0f;
    return;
  }
  const T* __restrict__ xu_row = static_cast<const T*>(p.XU) + ((size_t)chain * NT + t) * F;
  f4 xu[F / 4];
#pragma unroll
  for (int q = 0; q < F / 4; ++q) xu[q] = load4(xu_row + 4 * q);
  float* __restrict__ gam = gb + L.gam;
  float mx = -3.0e38f;
  for (int j = 0; j <= i; ++j) {
    f4 s4 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < F / 4; ++q) s4 += xu[q] * summ[j * (F / 4) + q];
    const float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    gam[(size_t)j * NT + t] = s;
    mx = fmaxf(mx, s);
  }
  float sum = 0.f;
  for (int j = 0; j <= i; ++j) {
    const float e = __expf(gam[(size_t)j * NT + t] - mx);
    gam[(size_t)j * NT + t] = e;
    sum += e;
  }
  const float inv = 1.0f / sum;
  for (int j = 0; j < i; ++j) gam[(size_t)j * NT + t] *= inv;
  gb[L.gcur + t] = gam[(size_t)i * NT + t] * inv;
}

// ------------------------------------------------------------------ R_j over a chunk
constexpr int kMemoWaves = 8;
constexpr int kMemoTilesPerWave = 2;
constexpr int kMemoChunkTiles = kMemoWaves * kMemoTilesPerWave;  // mini-batches (16 tokens each) per workgroup

template <typename T, int FT, int HTT> struct MemoShared {
  typename FragT<T>::type w1[FT * HTT][64];  // block (kb, ht): W1[16kb + 4g + j][16ht + n]
  typename FragT<T>::type w2[HTT * FT][64];  // block (ht, ct): W2[16ht + 4g + j][16ct + n]
  float b1[16 * HTT];
  float b2[16 * FT];
};

template <typename T, int FT, int HTT, bool BWD>
__global__ __launch_bounds__(64 * kMemoWaves) void memo_combine_kernel(MlpMemoParams p) {
  constexpr int F = 16 * FT;
  constexpr int FF = 16 * HTT;
  constexpr int K = 16;
  constexpr int NTW = kMemoTilesPerWave;
  constexpr int NB = FT * HTT / kMemoWaves;  // W1 (and W2) blocks each wave stages
  __shared__ MemoShared<T, FT, HTT> sh;

  // blockIdx -> (chain, chunk pair), the pairs of one chain on one XCD (shared
  // L2).  Chunk c needs about 2c+1 memo states, so a workgroup takes chunks c
  // and nchunk-1-c: every workgroup then does about the same work, which keeps
  // the in-order dispatch from waiting on a few long workgroups.
  const int npair = (p.nchunk + 1) >> 1;
  const int total = gridDim.x;
  int lin = blockIdx.x;
  if ((total & 7) == 0) lin = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int chain = lin / npair;
  const int pair = lin - chain * npair;
  const int h = chain % p.H;
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const MemoGateLayout L(NC, K, F, NS);

  const int wave = threadIdx.x >> 6;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  const size_t xoff = (size_t)chain * NT * F;
  const T* __restrict__ XQ = static_cast<const T*>(p.XQ) + xoff;
  float* __restrict__ gb = p.gates + (size_t)chain * L.stride;

#pragma unroll 1
  for (int half = 0; half < 2; ++half) {
    const int chunk = half == 0 ? pair : p.nchunk - 1 - pair;
    if (half == 1 && chunk == pair) break;  // (uniform: the middle chunk of an odd count)
    const int c0 = chunk * kMemoChunkTiles;                      // first mini-batch of the chunk
    const int clast = min(c0 + kMemoChunkTiles, NC) - 1;         // last mini-batch of the chunk
    const int jmax = clast / M;                                  // memo states 0..jmax-1 serve this chunk
    const int t0 = c0 + wave * NTW;                              // first mini-batch of this wave
    const int nv = max(0, min(NTW, NC - t0));                    // valid tiles of this wave
    const int tl = min(t0 + max(nv, 1) - 1, NC - 1);             // a valid tile index for padding

    // R_j = (XQ + ln_b) + ln_w * N_j with N_j the normalised rows of
    // gelu(XQ W1_j + b1_j) W2_j + b2_j.  The loop accumulates only the N_j terms:
    //   forward   acc_N = sum_{j<i} gamma_j N_j, and sum_{j<i} gamma_j = 1 - gamma_i
    //             multiplies (XQ + ln_b) once at the end;
    //   backward  dgamma_j = dOut . R_j = base + (dOut * ln_w) . N_j with the
    //             j-independent base = dOut . (XQ + ln_b) per token.
    Frag<T> xq[NTW][FT];  // XQ operand frags (free = token, k = feature)
    int seg[NTW];
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      const int tt = t < nv ? t0 + t : tl;
      seg[t] = t < nv ? tt / M : -1;
#pragma unroll
      for (int kb = 0; kb < FT; ++kb) xq[t][kb] = load_frag(XQ + (size_t)tt * K * F, F, 16 * kb);
    }

    f4 oacc[NTW][FT];  // forward: acc_N; backward: dOut * ln_w (C layout, token rows)
    f4 base[NTW];      // backward: dOut . (XQ + ln_b) of token rows 4g + j
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      base[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        if constexpr (BWD) {
          const size_t r0 = (size_t)(t < nv ? t0 + t : tl) * K * F + 16 * c + n;
          const T* d = static_cast<const T*>(p.dout) + xoff + r0;
          const float w = p.ln_w[h * F + 16 * c + n], b = p.ln_b[h * F + 16 * c + n];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float dv = (float)d[(4 * g + j) * F];
            oacc[t][c][j] = dv * w;
            base[t][j] += dv * ((float)XQ[r0 + (4 * g + j) * F] + b);
          }
        } else {
          oacc[t][c] = f4{0.f, 0.f, 0.f, 0.f};
        }
      }
      if constexpr (BWD) {
#pragma unroll
        for (int j = 0; j < 4; ++j) base[t][j] = sum_row16(base[t][j]);
      }
    }

    const float invF = 1.0f / (float)F;
#pragma unroll 1
    for (int jm = 0; jm < jmax; ++jm) {
      // ---- stage memo state jm (the previous state's reads are done); request
      //      this state's gates of the wave's tokens first (forward).  Each wave
      //      stages NB blocks of W1 and of W2, every load of a matrix issued
      //      before the first conversion.
      __syncthreads();
      f4 gjv[NTW];
      if constexpr (!BWD) {
#pragma unroll
        for (int t = 0; t < NTW; ++t)
          gjv[t] = *reinterpret_cast<const f4*>(gb + L.gam + (size_t)jm * NT + (t < nv ? t0 + t : tl) * K + 4 * g);
      }
      {
        const size_t st = (size_t)chain * NS + jm;
        const float* __restrict__ w1 = p.W1 + st * F * FF;
        const float* __restrict__ w2 = p.W2 + st * FF * F;
        f4 x[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int blk = wave + kMemoWaves * b, kb = blk / HTT, ht = blk - kb * HTT;
#pragma unroll
          for (int j = 0; j < 4; ++j) x[b][j] = w1[(16 * kb + 4 * g + j) * FF + 16 * ht + n];
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) sh.w1[wave + kMemoWaves * b][l] = to_frag<T>(x[b]).v;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int blk = wave + kMemoWaves * b, ht = blk / FT, ct = blk - ht * FT;
#pragma unroll
          for (int j = 0; j < 4; ++j) x[b][j] = w2[(16 * ht + 4 * g + j) * F + 16 * ct + n];
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) sh.w2[wave + kMemoWaves * b][l] = to_frag<T>(x[b]).v;
        for (int i = threadIdx.x; i < FF; i += 64 * kMemoWaves) sh.b1[i] = p.b1[st * FF + i];
        for (int i = threadIdx.x; i < F; i += 64 * kMemoWaves) sh.b2[i] = p.b2[st * F + i];
      }
      __syncthreads();

      bool any = false;
#pragma unroll
      for (int t = 0; t < NTW; ++t) any |= seg[t] > jm;
      if (!any) continue;  // (no barrier until the loop's next iteration, which every wave reaches)

      Tile acc[NTW][FT];  // Z2 + b2 (b2 rides in the accumulator)
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        const float b2 = sh.b2[16 * c + n];
#pragma unroll
        for (int t = 0; t < NTW; ++t) acc[t][c].v = f4{b2, b2, b2, b2};
      }
#pragma unroll 1
      for (int ht = 0; ht < HTT; ht += 2) {
        Frag<T> x2[2][NTW];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          Frag<T> w1f[FT];
#pragma unroll
          for (int kb = 0; kb < FT; ++kb) w1f[kb].v = sh.w1[kb * HTT + ht + hh][l];
          const f4 bias = *reinterpret_cast<const f4*>(&sh.b1[16 * (ht + hh) + 4 * g]);
#pragma unroll
          for (int t = 0; t < NTW; ++t) {
            Tile z;
            z.v = bias;  // b1 rides in the accumulator
#pragma unroll
            for (int kb = 0; kb < FT; kb += 2) mma32(z.v, w1f[kb], w1f[kb + 1], xq[t][kb], xq[t][kb + 1]);
            f4 a;
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = gelu_tanh(z.v[j]);
            x2[hh][t] = to_frag<T>(a);
          }
        }
        Frag<T> q0[FT], q1[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          q0[c].v = sh.w2[ht * FT + c][l];
          q1[c].v = sh.w2[(ht + 1) * FT + c][l];
        }
#pragma unroll
        for (int t = 0; t < NTW; ++t)
#pragma unroll
          for (int c = 0; c < FT; ++c) mma32(acc[t][c].v, x2[0][t], x2[1][t], q0[c], q1[c]);
      }

      // ---- N_jm = LN-normalised (Z2 + b2) per token row; fold it in
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        if (seg[t] <= jm) continue;
        f4 dg;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v[FT], s = 0.f;
#pragma unroll
          for (int c = 0; c < FT; ++c) {
            v[c] = acc[t][c].v[j];
            s += v[c];
          }
          const float mean = sum_row16(s) * invF;
          float q = 0.f;
#pragma unroll
          for (int c = 0; c < FT; ++c) {
            v[c] -= mean;
            q += v[c] * v[c];
          }
          const float rstd = rsqrt_f(sum_row16(q) * invF + p.eps);
          if constexpr (BWD) {
            float d = 0.f;
#pragma unroll
            for (int c = 0; c < FT; ++c) d += oacc[t][c][j] * v[c];
            dg[j] = base[t][j] + rstd * sum_row16(d);
          } else {
            const float gr = gjv[t][j] * rstd;
#pragma unroll
            for (int c = 0; c < FT; ++c) oacc[t][c][j] += gr * v[c];
          }
        }
        if constexpr (BWD) {
          const int tok0 = (t0 + t) * K + 4 * g;  // token of register j: tok0 + j
          if (n == 0) *reinterpret_cast<f4*>(gb + L.dgam + (size_t)jm * NT + tok0) = dg;
        }
      }
    }

    if constexpr (!BWD) {
      // out = gamma_i XQW + (1 - gamma_i)(XQ + ln_b) + ln_w acc_N  (segment 0:
      // gamma_i = 1 and acc_N = 0, so out = XQW)
      const T* __restrict__ XQW = static_cast<const T*>(p.XQW) + xoff;
      T* __restrict__ OUT = static_cast<T*>(p.out) + xoff;
      float lw[FT], lb[FT];
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        lw[c] = p.ln_w[h * F + 16 * c + n];
        lb[c] = p.ln_b[h * F + 16 * c + n];
      }
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        if (t >= nv) continue;
        const int tok0 = (t0 + t) * K + 4 * g;
        const f4 gc = *reinterpret_cast<const f4*>(gb + L.gcur + tok0);
#pragma unroll
        for (int c = 0; c < FT; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const size_t e = (size_t)(tok0 + j) * F + 16 * c + n;
            const float rest = seg[t] > 0 ? (1.0f - gc[j]) * ((float)XQ[e] + lb[c]) + lw[c] * oacc[t][c][j] : 0.0f;
            OUT[e] = (T)(gc[j] * (float)XQW[e] + rest);
          }
      }
    }
  }  // half
}

// ------------------------------------------------------------------ backward: softmax, dXU, dXQW
// one workgroup per (chain, block of kMemoThreads tokens), one token per thread
template <typename T, int F>
__global__ __launch_bounds__(kMemoThreads) void memo_finish_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  const int nblk = (p.NC * K + kMemoThreads - 1) / kMemoThreads;
  const int chain = blockIdx.x / nblk, blk = blockIdx.x - chain * nblk;
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const MemoGateLayout L(NC, K, F, NS);
  float* __restrict__ gb = p.gates + (size_t)chain * L.stride;
  __shared__ f4 summ[kMemoMaxStates * F / 4];
  const int t = blk * kMemoThreads + threadIdx.x;
  const int tmax = min(NT, (blk + 1) * kMemoThreads) - 1;
  const int ns = (tmax / K) / M + 1;
  for (int q = threadIdx.x; q < ns * F / 4; q += kMemoThreads)
    summ[q] = *reinterpret_cast<const f4*>(gb + L.summ + 4 * (size_t)q);
  __syncthreads();
  if (t >= NT) return;  // (no barrier follows)
  const size_t row = ((size_t)chain * NT + t) * F;
  const T* __restrict__ xqw_row = static_cast<const T*>(p.XQW) + row;
  const T* __restrict__ do_row = static_cast<const T*>(p.dout) + row;
  T* __restrict__ dxu_row = static_cast<T*>(p.dXU) + row;
  T* __restrict__ dxqw_row = static_cast<T*>(p.dXQW) + row;
  const int i = (t / K) / M;
  const float gc = gb[L.gcur + t];
  f4 dout[F / 4], dxu[F / 4];
  f4 dg4 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < F / 4; ++q) {
    dout[q] = load4(do_row + 4 * q);
    dg4 += dout[q] * load4(xqw_row + 4 * q);
    dxu[q] = f4{0.f, 0.f, 0.f, 0.f};
  }
  const float dgc = (dg4[0] + dg4[1]) + (dg4[2] + dg4[3]);
  float dscur = 0.f;  // d loss / d (XU . current summary)
  if (i > 0) {
    // softmax backward: dsims_j = gamma_j (dgamma_j - sum_k gamma_k dgamma_k)
    float S = gc * dgc;
    for (int j = 0; j < i; ++j) S += gb[L.gam + (size_t)j * NT + t] * gb[L.dgam + (size_t)j * NT + t];
    for (int j = 0; j <= i; ++j) {
      const float ds = j < i ? gb[L.gam + (size_t)j * NT + t] * (gb[L.dgam + (size_t)j * NT + t] - S)
                             : gc * (dgc - S);
#pragma unroll
      for (int q = 0; q < F / 4; ++q) dxu[q] += ds * summ[j * (F / 4) + q];
    }
    dscur = gc * (dgc - S);
  }
  gb[L.dscur + t] = dscur;
#pragma unroll
  for (int q = 0; q < F / 4; ++q) {
    store4(dxu_row + 4 * q, dxu[q]);
    store4(dxqw_row + 4 * q, gc * dout[q]);
  }
}

// one workgroup per (chain, segment): the summary's gradient (sum over the
// segment's tokens of dsims_current XU) spread evenly over the segment's
// tokens, dXK = that / (tokens in the segment); 0 for segment 0, whose
// summary is never a current one with gates (its dsims_current are 0).
template <typename T, int F>
__global__ __launch_bounds__(kSegThreads) void memo_dxk_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  __shared__ float part[kSegThreads];
  const int chain = blockIdx.x / p.NS, j = blockIdx.x - chain * p.NS;
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const MemoGateLayout L(NC, K, F, NS);
  const float* __restrict__ ds = p.gates + (size_t)chain * L.stride + L.dscur;
  const T* __restrict__ XU = static_cast<const T*>(p.XU) + (size_t)chain * NT * F;
  T* __restrict__ DXK = static_cast<T*>(p.dXK) + (size_t)chain * NT * F;
  const int t0 = j * M * K, t1 = min((j + 1) * M, NC) * K;
  const float tot = segment_column_sum<T, F>(XU, t0, t1, [ds](int t) { return ds[t]; }, part);
  const T v = (T)(tot / (float)(t1 - t0));
  for (int t = t0 + (int)threadIdx.x / F; t < t1; t += kSegThreads / F) DXK[(size_t)t * F + threadIdx.x % F] = v;
}

// ------------------------------------------------------------------ launchers
template <typename T, int FT, int HTT>
static hipError_t launch_memo_t(const MlpMemoParams& p, bool bwd, hipStream_t stream) {
  const dim3 grid(p.B * p.H * ((p.nchunk + 1) / 2)), block(64 * kMemoWaves);
  const int nblk = (p.NC * 16 + kMemoThreads - 1) / kMemoThreads;
  if (bwd) {
    hipLaunchKernelGGL((memo_combine_kernel<T, FT, HTT, true>), grid, block, 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((memo_finish_kernel<T, 16 * FT>), dim3(p.B * p.H * nblk), dim3(kMemoThreads), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((memo_dxk_kernel<T, 16 * FT>), dim3(p.B * p.H * p.NS), dim3(kSegThreads), 0, stream, p);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((memo_summary_kernel<T, 16 * FT>), dim3(p.B * p.H * p.NS), dim3(kSegThreads), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((memo_gate_kernel<T, 16 * FT>), dim3(p.B * p.H * nblk), dim3(kMemoThreads), 0, stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((memo_combine_kernel<T, FT, HTT, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <typename T, int FT>
static hipError_t launch_memo_f(const MlpMemoParams& p, bool bwd, hipStream_t stream) {
  switch (p.FF) {
    case 64: return launch_memo_t<T, FT, 4>(p, bwd, stream);
    case 128: return launch_memo_t<T, FT, 8>(p, bwd, stream);
    case 256: return launch_memo_t<T, FT, 16>(p, bwd, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_mlp_memo(const MlpMemoParams& p, int dtype, bool bwd, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_memo_f<__bf16, 4>(p, bwd, stream);
    if (p.F == 32) return launch_memo_f<__bf16, 2>(p, bwd, stream);
  } else {
    if (p.F == 64) return launch_memo_f<float, 4>(p, bwd, stream);
    if (p.F == 32) return launch_memo_f<float, 2>(p, bwd, stream);
  }
  return hipErrorInvalidValue;
}

int mlp_memo_chunk_tiles() { return kMemoChunkTiles; }

}  // namespace ttt
