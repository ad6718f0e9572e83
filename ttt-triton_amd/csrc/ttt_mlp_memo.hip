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
//   memo_gate_kernel      one workgroup per 64 tokens: the gates (written as
//                         gamma^T [NS][tokens] plus the current-segment gate);
//   memo_combine_kernel   one workgroup per (chain, pair of 256-token chunks,
//                         or 128-token ones where the pairs would leave CUs
//                         idle: 128 -> 256 workgroups for the forecaster's
//                         combines, 63-78 -> 38-48 us):
//                         for each memo state j below a chunk's last segment, stage
//                         W1_j/W2_j into LDS in MFMA operand order (as the cached
//                         readout does), run the chunk's tiles of later
//                         segments through R_j and accumulate gamma_j R_j (forward)
//                         or dOut . R_j (backward: the gate gradients);
//   memo_finish_kernel    (backward) one workgroup per 64 tokens: the softmax
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
#include "ttt_buf.h"
#include "ttt_fixed_mlp.h"
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

// Sum over a segment's tokens t0..t1-1 of w(t) * X[t][f]: each thread reads
// 4 consecutive features of a row (one 8- or 16-byte load), kSegThreads / (F/4)
// rows at a time; the block's total for column f = threadIdx.x % F is returned
// to every thread of that column.  `part` holds kSegPart floats.
constexpr int kSegPart = 4 * kSegThreads;
template <typename T, int F, typename W>
__device__ __forceinline__ float segment_column_sum(const T* __restrict__ X, int t0, int t1, W w, float* part) {
  constexpr int C = F / 4, R = kSegThreads / C;  // threads per row, rows per pass
  static_assert(R * F <= kSegPart, "partials fit");
  const int c = threadIdx.x % C, r = threadIdx.x / C;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int t = t0 + r; t < t1; t += R) acc += w(t) * load4(X + (size_t)t * F + 4 * c);
  *reinterpret_cast<f4*>(&part[r * F + 4 * c]) = acc;
  __syncthreads();
  const int f = threadIdx.x % F;
  float tot = 0.f;
#pragma unroll
  for (int q = 0; q < R; ++q) tot += part[q * F + f];
  return tot;
}

// one workgroup per (chain, segment): mean of XK over the segment
template <typename T, int F>
__global__ __launch_bounds__(kSegThreads) void memo_summary_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  __shared__ __align__(16) float part[kSegPart];
  const int chain = blockIdx.x / p.NS, j = blockIdx.x - chain * p.NS;
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const MemoGateLayout L(NC, K, F, NS);
  const T* __restrict__ XK = static_cast<const T*>(p.XK) + (size_t)chain * NT * F;
  const int t0 = j * M * K, t1 = min((j + 1) * M, NC) * K;
  const float tot = segment_column_sum<T, F>(XK, t0, t1, [](int) { return 1.0f; }, part);
  if (threadIdx.x < F) p.gates[(size_t)chain * L.stride + L.summ + (size_t)j * F + threadIdx.x] = tot / (float)(t1 - t0);
}

// Gate and finish kernels: a workgroup of kMemoThreads threads takes
// kTokBlk consecutive tokens of one chain and works in two layouts:
//   token-major  thread (sub = wave, tk = lane): token tk, segments j = sub,
//                sub + 4, ...  Loads of per-(segment, token) gate data
//                gam[j][t] are then coalesced over the wave's 64 tokens;
//   row          the 16 lanes of a DPP row share a token (kRowUnroll tokens
//                per row) and hold F/16 consecutive features each, so token
//                rows are read and written as contiguous segments.
// Summaries are staged per chunk of kSegChunk segments in LDS and read as
// broadcasts (every lane of a wave at the same segment).  Chunks of 16 keep
// the workgroups' LDS small enough for five per CU (the gate kernel's
// registers are held to that occupancy too): finish 84 -> 76 us, gate
// 52 -> 46 us at B16 H12 T2048 with 16 segments.  The finish kernel requests
// every load of the first chunk up front (76 -> 67 us; it then holds 116
// registers, four workgroups per CU: capped at five it spills and is slower);
// the gate kernel keeps the first chunk's logits in registers for its second
// pass (46 -> 37 us, the same with or without its cap).
constexpr int kTokBlk = 64;
constexpr int kRowUnroll = kTokBlk / (kMemoThreads / 16);
constexpr int kSegChunk = 16;

template <int F> using RowVec = std::conditional_t<F / 16 == 4, f4, f2>;

template <int F>
__device__ __forceinline__ void stage_summaries(float (*sm)[F], const float* __restrict__ summ, int c, int NS) {
  const int n = min(kSegChunk, NS - c * kSegChunk) * F;
  const float* src = summ + (size_t)c * kSegChunk * F;
  for (int idx = threadIdx.x; idx < n; idx += kMemoThreads) sm[idx / F][idx % F] = src[idx];
}

// The gates: logits s_j = XU_t . summary_j for j = 0..i and gamma =
// softmax(s).  Each thread keeps an online (max, sum) over its segments, the
// four partial pairs of a token are merged through LDS, and a second pass
// writes the normalised gates: the first chunk's logits kept in registers,
// later chunks' recomputed (the same operations, so the same value).
template <typename T, int F>
__global__ __launch_bounds__(kMemoThreads, 5) void memo_gate_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  constexpr int FPL = F / 16;
  constexpr int NSUB = kMemoThreads / 64;
  // XU rows in fp32, padded (the column reads of 32 rows reach 32 banks) and
  // column f at f ^ ((f >> 4) & 2) (the row writes of 16 threads, four
  // columns each, reach 32 banks: columns f and f + 32 of one row would share
  // one at F = 64)
  __shared__ float xs[kTokBlk][F + 1];
  auto xcol = [](int f) { return f ^ ((f >> 4) & 2); };
  __shared__ __align__(16) float sm[kSegChunk][F];
  __shared__ float red[2][NSUB][kTokBlk];
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const int nblk = (NT + kTokBlk - 1) / kTokBlk;
  const int chain = blockIdx.x / nblk, blk = blockIdx.x - chain * nblk;
  const MemoGateLayout L(NC, K, F, NS);
  float* __restrict__ gb = p.gates + (size_t)chain * L.stride;
  const float* __restrict__ summ = gb + L.summ;
  float* __restrict__ gam = gb + L.gam;
  const int tb = blk * kTokBlk;
  const int ilast = ((min(tb + kTokBlk, NT) - 1) / K) / M;  // the block's largest segment index
  const int nch = ilast / kSegChunk + 1;

  {  // XU rows -> LDS (row layout)
    const int q = threadIdx.x & 15, row = threadIdx.x >> 4;
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int tk = u * (kMemoThreads / 16) + row;
      float x[FPL];
      load_n<FPL>(static_cast<const T*>(p.XU) + ((size_t)chain * NT + min(tb + tk, NT - 1)) * F + FPL * q, x);
#pragma unroll
      for (int k = 0; k < FPL; ++k) xs[tk][xcol(FPL * q + k)] = x[k];
    }
  }
  const int sub = threadIdx.x >> 6, tk = threadIdx.x & 63;
  const int t = tb + tk;
  const int i = t < NT ? (t / K) / M : -1;
  stage_summaries<F>(sm, summ, 0, NS);
  __syncthreads();
  float x[F];
#pragma unroll
  for (int f = 0; f < F; ++f) x[f] = xs[tk][xcol(f)];
  auto logit = [&](int jj) {
    const f4* sj = reinterpret_cast<const f4*>(sm[jj]);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < F / 4; ++k) {
      const f4 v = sj[k];
      s += x[4 * k] * v[0] + x[4 * k + 1] * v[1] + x[4 * k + 2] * v[2] + x[4 * k + 3] * v[3];
    }
    return s;
  };
  constexpr int KC = kSegChunk / NSUB;  // first-chunk segments per thread
  float lg[KC];                         // their logits
  float m = -3.0e38f, l = 0.f;
  auto online = [&](float sj) {
    const float mn = fmaxf(m, sj);
    l = l * __expf(m - mn) + __expf(sj - mn);
    m = mn;
  };
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    lg[k] = 0.f;
    if (sub + NSUB * k <= i) {
      lg[k] = logit(sub + NSUB * k);
      online(lg[k]);
    }
  }
  for (int c = 1; c < nch; ++c) {
    __syncthreads();
    stage_summaries<F>(sm, summ, c, NS);
    __syncthreads();
    for (int jj = sub; jj < kSegChunk && c * kSegChunk + jj <= i; jj += NSUB) online(logit(jj));
  }
  red[0][sub][tk] = m;
  red[1][sub][tk] = l;
  __syncthreads();
  float mx = red[0][0][tk];
#pragma unroll
  for (int u = 1; u < NSUB; ++u) mx = fmaxf(mx, red[0][u][tk]);
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < NSUB; ++u) sum += red[1][u][tk] * __expf(red[0][u][tk] - mx);
  const float inv = i >= 0 ? 1.0f / sum : 0.f;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int j = sub + NSUB * k;
    if (j <= i) {
      const float gj = __expf(lg[k] - mx) * inv;
      gam[(size_t)j * NT + t] = gj;
      if (j == i) gb[L.gcur + t] = gj;
    }
  }
  for (int c = 1; c < nch; ++c) {
    __syncthreads();
    stage_summaries<F>(sm, summ, c, NS);
    __syncthreads();
    for (int jj = sub; jj < kSegChunk && c * kSegChunk + jj <= i; jj += NSUB) {
      const int j = c * kSegChunk + jj;
      const float gj = __expf(logit(jj) - mx) * inv;
      gam[(size_t)j * NT + t] = gj;
      if (j == i) gb[L.gcur + t] = gj;
    }
  }
}

// ------------------------------------------------------------------ R_j over a chunk
constexpr int kMemoWaves = 8;
constexpr int kMemoTilesPerWave = 2;
constexpr int kMemoChunkTiles = kMemoWaves * kMemoTilesPerWave;  // mini-batches (16 tokens each) per workgroup
constexpr int kComputeUnits = 256;  // MI355X

// Packed memo states (bf16): each state's LDS image -- the FixedMlpLds struct
// the staging builds, operand frags and biases -- written once by
// memo_pack_kernel, padded to whole kilobytes so that a wave copies it 1 KB
// (64 lanes x 16 bytes) at a time with direct-to-LDS loads.
template <typename T, int FT, int HTT> constexpr int kMemoImg = (int)((sizeof(FixedMlpLds<T, FT, HTT>) + 1023) & ~1023);

// one workgroup per (chain, state): stage the state as the combiner would,
// then copy the LDS image out
template <typename T, int FT, int HTT>
__global__ __launch_bounds__(256) void memo_pack_kernel(MlpMemoParams p) {
  constexpr int F = 16 * FT, FF = 16 * HTT, IMG = kMemoImg<T, FT, HTT>;
  __shared__ __align__(16) unsigned char img[IMG];
  auto& sh = *reinterpret_cast<FixedMlpLds<T, FT, HTT>*>(img);
  const size_t st = blockIdx.x;  // chain * NS + state
  stage_fixed_mlp<T, FT, HTT, 4>(sh, p.W1 + st * F * FF, p.b1 + st * FF, p.W2 + st * FF * F, p.b2 + st * F);
  __syncthreads();
  const u4v* src = reinterpret_cast<const u4v*>(img);
  u4v* dst = reinterpret_cast<u4v*>(p.packed + st * IMG);
  for (int i = threadIdx.x; i < IMG / 16; i += 256) dst[i] = src[i];
}

template <typename T, int FT, int HTT, bool BWD, bool PK, int NTW>
__global__ __launch_bounds__(64 * kMemoWaves) void memo_combine_kernel(MlpMemoParams p) {
  constexpr int F = 16 * FT;
  constexpr int FF = 16 * HTT;
  constexpr int K = 16;
  constexpr int CT = kMemoWaves * NTW;  // mini-batches per chunk
  constexpr int IMG = kMemoImg<T, FT, HTT>;
  // unpacked: one staging area, filled between two barriers per state;
  // packed: two images, the next state's copied in while the current one is used
  __shared__ __align__(16) unsigned char lds[PK ? 2 * IMG : (int)sizeof(FixedMlpLds<T, FT, HTT>)];

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
    const int c0 = chunk * CT;                                   // first mini-batch of the chunk
    const int clast = min(c0 + CT, NC) - 1;                      // last mini-batch of the chunk
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

    // Token-major throughout (the layout of the xq frags and of the fixed MLP's
    // Z2): lane (g, n) holds features 16c + 4g + j of token n of each tile.
    f4 lw[FT], lb[FT];  // ln_w, ln_b of those features
#pragma unroll
    for (int c = 0; c < FT; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lw[c][j] = p.ln_w[h * F + 16 * c + 4 * g + j];
        lb[c][j] = p.ln_b[h * F + 16 * c + 4 * g + j];
      }
    f4 oacc[NTW][FT];  // forward: acc_N; backward: dOut * ln_w
    float base[NTW];   // backward: dOut . (XQ + ln_b) of token n
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      base[t] = 0.f;
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        if constexpr (BWD) {
          const size_t e = ((size_t)(t < nv ? t0 + t : tl) * K + n) * F + 16 * c + 4 * g;
          const f4 dv = load4(static_cast<const T*>(p.dout) + xoff + e);
          const f4 xb = frag_to_f4(xq[t][c]) + lb[c];
          oacc[t][c] = dv * lw[c];
          base[t] += (dv[0] * xb[0] + dv[1] * xb[1]) + (dv[2] * xb[2] + dv[3] * xb[3]);
        } else {
          oacc[t][c] = f4{0.f, 0.f, 0.f, 0.f};
        }
      }
      if constexpr (BWD) base[t] = sum_col4(base[t]);
    }

    const float invF = 1.0f / (float)F;
    // packed: copy state jm's image into buffer b, 1 KB per wave and copy
    auto dma_state = [&](int jm, int b) {
      const unsigned char* src = p.packed + ((size_t)chain * NS + jm) * IMG + 16 * l;
      for (int c = wave; c < IMG / 1024; c += kMemoWaves)
        __builtin_amdgcn_global_load_lds(src + c * 1024, (__attribute__((address_space(3))) void*)(lds + b * IMG + c * 1024),
                                         16, 0, 0);
    };
    if constexpr (PK) {
      __syncthreads();  // (the other chunk's last reads of the buffers are done)
      if (jmax > 0) dma_state(0, 0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
#pragma unroll 1
    for (int jm = 0; jm < jmax; ++jm) {
      // ---- memo state jm in LDS.  This state's gates of the wave's tokens are
      //      requested first (forward).  Unpacked: each wave stages NB blocks
      //      of W1 and of W2 and a share of the biases between two barriers,
      //      every load issued before the first conversion, so that a state
      //      costs one memory latency.  Packed: state jm's image arrived during
      //      the previous state; state jm + 1's copy is requested now, into the
      //      buffer the previous state used.
      if constexpr (!PK) __syncthreads();
      float gjv[NTW];  // gamma_jm of token n
      if constexpr (!BWD) {
#pragma unroll
        for (int t = 0; t < NTW; ++t) gjv[t] = gb[L.gam + (size_t)jm * NT + (t < nv ? t0 + t : tl) * K + n];
      }
      if constexpr (PK) {
        if (jm + 1 < jmax) dma_state(jm + 1, (jm + 1) & 1);
      } else {
        const size_t st = (size_t)chain * NS + jm;
        stage_fixed_mlp<T, FT, HTT, kMemoWaves>(*reinterpret_cast<FixedMlpLds<T, FT, HTT>*>(lds), p.W1 + st * F * FF,
                                                p.b1 + st * FF, p.W2 + st * FF * F, p.b2 + st * F);
        __syncthreads();
      }
      const auto& sh = *reinterpret_cast<const FixedMlpLds<T, FT, HTT>*>(lds + (PK ? (jm & 1) * IMG : 0));

      bool any = false;
#pragma unroll
      for (int t = 0; t < NTW; ++t) any |= seg[t] > jm;
      if (!any) {
        if constexpr (PK) {
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
        }
        continue;  // (unpacked: no barrier until the loop's next iteration, which every wave reaches)
      }

      Tile acc[NTW][FT];  // Z2 + b2
      fixed_mlp_tiles<T, FT, HTT, NTW>(sh, xq, acc);

      // ---- N_jm = LN-normalised (Z2 + b2) per token row (its features in
      //      lanes n, n + 16, n + 32, n + 48: sum_col4); fold it in
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        if (seg[t] <= jm) continue;
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < FT; ++c) s += (acc[t][c].v[0] + acc[t][c].v[1]) + (acc[t][c].v[2] + acc[t][c].v[3]);
        const float mean = sum_col4(s) * invF;
        float q = 0.f;
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          acc[t][c].v -= mean;
          const f4 v = acc[t][c].v;
          q += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
        }
        const float rstd = rsqrt_f(sum_col4(q) * invF + p.eps);
        if constexpr (BWD) {
          float d = 0.f;
#pragma unroll
          for (int c = 0; c < FT; ++c) {
            const f4 v = acc[t][c].v, o = oacc[t][c];
            d += (o[0] * v[0] + o[1] * v[1]) + (o[2] * v[2] + o[3] * v[3]);
          }
          const float dg = base[t] + rstd * sum_col4(d);
          if (g == 0) gb[L.dgam + (size_t)jm * NT + (t0 + t) * K + n] = dg;
        } else {
          const float gr = gjv[t] * rstd;
#pragma unroll
          for (int c = 0; c < FT; ++c) oacc[t][c] += gr * acc[t][c].v;
        }
      }
      if constexpr (PK) {
        // state jm + 1's image complete in every wave; state jm's buffer free
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }

    if constexpr (!BWD) {
      // out = gamma_i XQW + (1 - gamma_i)(XQ + ln_b) + ln_w acc_N  (segment 0:
      // gamma_i = 1 and acc_N = 0, so out = XQW)
      const T* __restrict__ XQW = static_cast<const T*>(p.XQW) + xoff;
      T* __restrict__ OUT = static_cast<T*>(p.out) + xoff;
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        if (t >= nv) continue;
        const int tok = (t0 + t) * K + n;
        const float gc = gb[L.gcur + tok];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          const size_t e = (size_t)tok * F + 16 * c + 4 * g;
          const f4 rest = seg[t] > 0 ? (1.0f - gc) * (frag_to_f4(xq[t][c]) + lb[c]) + lw[c] * oacc[t][c]
                                     : f4{0.f, 0.f, 0.f, 0.f};
          store4(OUT + e, gc * load4(XQW + e) + rest);
        }
      }
    }
  }  // half
}

// ------------------------------------------------------------------ backward: softmax, dXU, dXQW
// Layouts as in the gate kernel.  dsims_j = gamma_j (dgamma_j - S) with
// S = sum_{k<=i} gamma_k dgamma_k: the token-major threads sum their segments'
// gamma_j dgamma_j (coalesced loads), the four partials of a token meet in
// LDS, and per chunk of segments the dsims go to LDS, from where the row
// layout accumulates dXU = sum_{j<i} dsims_j summ_j + dsims_i summ_i with
// broadcast reads only.
template <typename T, int F>
__global__ __launch_bounds__(kMemoThreads) void memo_finish_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  constexpr int FPL = F / 16;
  constexpr int NSUB = kMemoThreads / 64;
  constexpr int U = kRowUnroll;
  using VT = RowVec<F>;
  __shared__ __align__(16) float sm[kSegChunk][F];
  __shared__ float dsl[kTokBlk][kSegChunk + 1];
  __shared__ float sp[NSUB][kTokBlk];
  __shared__ float dgl[kTokBlk];
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const int nblk = (NT + kTokBlk - 1) / kTokBlk;
  const int chain = blockIdx.x / nblk, blk = blockIdx.x - chain * nblk;
  const MemoGateLayout L(NC, K, F, NS);
  float* __restrict__ gb = p.gates + (size_t)chain * L.stride;
  const float* __restrict__ gam = gb + L.gam;
  const float* __restrict__ dgam = gb + L.dgam;
  const float* __restrict__ summ = gb + L.summ;
  const int tb = blk * kTokBlk;
  const int ilast = ((min(tb + kTokBlk, NT) - 1) / K) / M;
  const int nch = (ilast + kSegChunk - 1) / kSegChunk;  // chunks of segments below the block's last one

  // Every load the first chunk of segments needs is requested before the
  // first use of any (one memory latency for the common case NS <= 16): the
  // token-major gates of chunk 0 kept in registers, chunk 0's summaries into
  // LDS, the row layout's dOut, XQW, current gate and current summary.
  constexpr int KC = kSegChunk / NSUB;  // chunk-0 segments per token-major thread
  const int sub = threadIdx.x >> 6, tk = threadIdx.x & 63;
  const int tc = min(tb + tk, NT - 1);
  const int i = (tc / K) / M;
  const float gc = gb[L.gcur + tc];
  float ga[KC], dga[KC];  // gamma_j, dgamma_j of segments j = sub + NSUB k of chunk 0 (0 past i)
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int j = sub + NSUB * k;
    ga[k] = j < i ? gam[(size_t)j * NT + tc] : 0.f;
    dga[k] = j < i ? dgam[(size_t)j * NT + tc] : 0.f;
  }
  if (nch > 0) stage_summaries<F>(sm, summ, 0, NS);

  // ---- row layout: dOut, the current gate, dgamma_current = dOut . XQW
  const int q = threadIdx.x & 15, row = threadIdx.x >> 4;
  const int f0 = FPL * q;
  float dout[U][FPL], gcr[U];
  VT svc[U];  // the current summary (segment iu) of each row's token
  int iu[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tkr = u * (kMemoThreads / 16) + row;
    const int tcr = min(tb + tkr, NT - 1);  // tokens past the end compute on the last one and store nothing
    iu[u] = (tcr / K) / M;
    float xqw[FPL];
    const size_t e = ((size_t)chain * NT + tcr) * F + f0;
    load_n<FPL>(static_cast<const T*>(p.dout) + e, dout[u]);
    load_n<FPL>(static_cast<const T*>(p.XQW) + e, xqw);
    gcr[u] = gb[L.gcur + tcr];
    svc[u] = *reinterpret_cast<const VT*>(summ + (size_t)iu[u] * F + f0);
    float dg = 0.f;
#pragma unroll
    for (int k = 0; k < FPL; ++k) dg += dout[u][k] * xqw[k];
    dg = sum_row16(dg);
    if (q == 0) dgl[tkr] = dg;
  }

  // ---- token-major: S
  {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < KC; ++k) s += ga[k] * dga[k];
    for (int j = kSegChunk + sub; j < i; j += NSUB) s += gam[(size_t)j * NT + tc] * dgam[(size_t)j * NT + tc];
    sp[sub][tk] = s;
  }
  __syncthreads();
  const float dgc = dgl[tk];
  float S = gc * dgc;
#pragma unroll
  for (int u = 0; u < NSUB; ++u) S += sp[u][tk];
  const float dscur = i > 0 ? gc * (dgc - S) : 0.f;  // d loss / d (XU . current summary)
  if (sub == 0 && tb + tk < NT) gb[L.dscur + tb + tk] = dscur;

  float dxu[U][FPL];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int k = 0; k < FPL; ++k) dxu[u][k] = 0.f;
  for (int c = 0; c < nch; ++c) {
    if (c > 0) {
      __syncthreads();  // the previous chunk's LDS reads are done
      stage_summaries<F>(sm, summ, c, NS);
      for (int jj = sub; jj < kSegChunk && c * kSegChunk + jj < i; jj += NSUB) {
        const int j = c * kSegChunk + jj;
        dsl[tk][jj] = gam[(size_t)j * NT + tc] * (dgam[(size_t)j * NT + tc] - S);
      }
    } else {
#pragma unroll
      for (int k = 0; k < KC; ++k)
        if (sub + NSUB * k < i) dsl[tk][sub + NSUB * k] = ga[k] * (dga[k] - S);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int tkr = u * (kMemoThreads / 16) + row;
      const int n = min(kSegChunk, iu[u] - c * kSegChunk);  // (uniform over the row)
#pragma unroll 4
      for (int jj = 0; jj < n; ++jj) {
        const float ds = dsl[tkr][jj];
        const VT sv = *reinterpret_cast<const VT*>(&sm[jj][f0]);
#pragma unroll
        for (int k = 0; k < FPL; ++k) dxu[u][k] += ds * sv[k];
      }
    }
  }
  __syncthreads();
  sp[0][tk] = dscur;  // (sub 0..3 write the same value)
  __syncthreads();

  // ---- row layout: the current segment's term and the stores
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tkr = u * (kMemoThreads / 16) + row;
    if (tb + tkr >= NT) continue;  // (uniform over the row)
    const size_t e = ((size_t)chain * NT + tb + tkr) * F + f0;
    if (iu[u] > 0) {
      const float dsc = sp[0][tkr];
#pragma unroll
      for (int k = 0; k < FPL; ++k) dxu[u][k] += dsc * svc[u][k];
    }
    float dq[FPL];
#pragma unroll
    for (int k = 0; k < FPL; ++k) dq[k] = gcr[u] * dout[u][k];
    store_n<FPL>(static_cast<T*>(p.dXU) + e, dxu[u]);
    store_n<FPL>(static_cast<T*>(p.dXQW) + e, dq);
  }
}

// one workgroup per (chain, segment): the summary's gradient (sum over the
// segment's tokens of dsims_current XU) spread evenly over the segment's
// tokens, dXK = that / (tokens in the segment); 0 for segment 0, whose
// summary is never a current one with gates (its dsims_current are 0).
template <typename T, int F>
__global__ __launch_bounds__(kSegThreads) void memo_dxk_kernel(MlpMemoParams p) {
  constexpr int K = 16;
  __shared__ __align__(16) float part[kSegPart];
  const int chain = blockIdx.x / p.NS, j = blockIdx.x - chain * p.NS;
  const int NC = p.NC, M = p.M, NS = p.NS, NT = NC * K;
  const MemoGateLayout L(NC, K, F, NS);
  const float* __restrict__ ds = p.gates + (size_t)chain * L.stride + L.dscur;
  const T* __restrict__ XU = static_cast<const T*>(p.XU) + (size_t)chain * NT * F;
  T* __restrict__ DXK = static_cast<T*>(p.dXK) + (size_t)chain * NT * F;
  const int t0 = j * M * K, t1 = min((j + 1) * M, NC) * K;
  const float tot = segment_column_sum<T, F>(XU, t0, t1, [ds](int t) { return ds[t]; }, part);
  __syncthreads();  // every thread's partial sums read
  if (threadIdx.x < F) part[threadIdx.x] = tot / (float)(t1 - t0);
  __syncthreads();
  // the same row for every token of the segment, 4 features per thread
  constexpr int C = F / 4;
  const int c = threadIdx.x % C;
  const f4 v = *reinterpret_cast<const f4*>(&part[4 * c]);
  for (int t = t0 + (int)threadIdx.x / C; t < t1; t += kSegThreads / C) store4(DXK + (size_t)t * F + 4 * c, v);
}

// ------------------------------------------------------------------ launchers
template <typename T, int FT, int HTT, bool BWD, int NTW>
static hipError_t launch_combine_n(const MlpMemoParams& p, hipStream_t stream) {
  const dim3 grid(p.B * p.H * ((p.nchunk + 1) / 2)), block(64 * kMemoWaves);
  if constexpr (sizeof(T) == 2) {
    if (p.packed != nullptr) {
      hipLaunchKernelGGL((memo_combine_kernel<T, FT, HTT, BWD, true, NTW>), grid, block, 0, stream, p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((memo_combine_kernel<T, FT, HTT, BWD, false, NTW>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <typename T, int FT, int HTT, bool BWD>
static hipError_t launch_combine(const MlpMemoParams& p, hipStream_t stream) {
  // p.nchunk was set from the same chunk size
  if (mlp_memo_chunk_tiles(p.B, p.H, p.NC) == kMemoWaves) return launch_combine_n<T, FT, HTT, BWD, 1>(p, stream);
  return launch_combine_n<T, FT, HTT, BWD, kMemoTilesPerWave>(p, stream);
}

template <typename T, int FT, int HTT>
static hipError_t launch_memo_t(const MlpMemoParams& p, bool bwd, hipStream_t stream) {
  const int nrow = (p.NC * 16 + kTokBlk - 1) / kTokBlk;  // workgroups per chain of the gate and finish kernels
  if (bwd) {
    hipError_t e = launch_combine<T, FT, HTT, true>(p, stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((memo_finish_kernel<T, 16 * FT>), dim3(p.B * p.H * nrow), dim3(kMemoThreads), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((memo_dxk_kernel<T, 16 * FT>), dim3(p.B * p.H * p.NS), dim3(kSegThreads), 0, stream, p);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((memo_summary_kernel<T, 16 * FT>), dim3(p.B * p.H * p.NS), dim3(kSegThreads), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((memo_gate_kernel<T, 16 * FT>), dim3(p.B * p.H * nrow), dim3(kMemoThreads), 0, stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if constexpr (sizeof(T) == 2) {
    if (p.packed != nullptr) {
      hipLaunchKernelGGL((memo_pack_kernel<T, FT, HTT>), dim3(p.B * p.H * p.NS), dim3(256), 0, stream, p);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  return launch_combine<T, FT, HTT, false>(p, stream);
}

template <typename T, int FT>
static hipError_t launch_memo_f(const MlpMemoParams& p, bool bwd, hipStream_t stream) {
  switch (p.FF) {
    case 32: return launch_memo_t<T, FT, 2>(p, bwd, stream);
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
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_memo_f<_Float16, 4>(p, bwd, stream);
    if (p.F == 32) return launch_memo_f<_Float16, 2>(p, bwd, stream);
  } else {
    if (p.F == 64) return launch_memo_f<float, 4>(p, bwd, stream);
    if (p.F == 32) return launch_memo_f<float, 2>(p, bwd, stream);
  }
  return hipErrorInvalidValue;
}

// Mini-batches per combiner chunk: two tiles per wave, or one where the
// pairs of two-tile chunks would leave CUs idle (few chains or short
// sequences, e.g. the forecaster's 128 chains of 32 mini-batches).
int mlp_memo_chunk_tiles(int B, int H, int NC) {
  const long long pairs = (long long)B * H * (((NC + kMemoChunkTiles - 1) / kMemoChunkTiles + 1) / 2);
  return pairs < kComputeUnits ? kMemoWaves : kMemoChunkTiles;
}

size_t mlp_memo_image_bytes(int F, int FF) {
  const int FT = F / 16;
  switch (FF) {
    case 32: return FT == 4 ? kMemoImg<__bf16, 4, 2> : kMemoImg<__bf16, 2, 2>;
    case 64: return FT == 4 ? kMemoImg<__bf16, 4, 4> : kMemoImg<__bf16, 2, 4>;
    case 128: return FT == 4 ? kMemoImg<__bf16, 4, 8> : kMemoImg<__bf16, 2, 8>;
    case 256: return FT == 4 ? kMemoImg<__bf16, 4, 16> : kMemoImg<__bf16, 2, 16>;
    default: return 0;
  }
}
// one image size for both 16-bit activation types
static_assert(kMemoImg<_Float16, 4, 16> == kMemoImg<__bf16, 4, 16> && kMemoImg<_Float16, 2, 2> == kMemoImg<__bf16, 2, 2>,
              "fp16 and bf16 memo images differ in size");

}  // namespace ttt
