// Fixed-weight TTT-MLP readout on gfx950:
//   out = XQ + LN_eps(gelu(XQ W1 + b1) W2 + b2)      (no state update)
// for every token of a segment, with one (W1, b1, W2, b2) per (batch, head)
// chain (kernels/mlp_cached_readout.py:88-109,143, indexed per chain).
//
// The weights are fixed, so tokens are independent: a workgroup of eight waves
// takes one chain and a chunk of up to 512 tokens.  It stages the chain's W1
// and W2 once into LDS, already in MFMA operand order (one 4-element vector
// per lane per 16x16 block, so every operand read is one conflict-free
// ds_read), then each wave runs two rounds of up to two 16-token tiles
// (two rounds per staging: 61 -> 58 us at B16 H12 T2048; four: 69) through
//
//   Z1^T = W1^T XQ^T           (hidden x token: its C layout is the B operand
//   X2^T = gelu(Z1^T + b1)      of the next product with no transpose)
//   Z2^T = W2^T X2^T + b2       accumulated over hidden tiles two at a time
//   out  = XQ + ln_w * (Z2 - mean) / sqrt(var + eps) + ln_b
//
// Z2 arrives token-major (lane (g, n): token n, features 16c + 4g + j), the
// layout of the XQ operand frags and of a 16-byte row store: the LayerNorm
// takes its row sums over four lanes (two lane swaps) and the residual and
// the store need no transpose.
//
// W is read from HBM once per workgroup; blocks are mapped so that the chunks
// of one chain run on one XCD and share its L2.  Two workgroups fit a CU's LDS
// and the waves stay within 128 registers, so each SIMD interleaves four
// waves (measured 5% faster at B16 H12 T2048 than four waves of four tiles).
#include "ttt_fixed_mlp.h"
#include "ttt_kernels.h"

namespace ttt {

template <typename T, int FT, int HTT> struct ReadoutShared {
  FixedMlpLds<T, FT, HTT> w;
  alignas(16) float lnw[16 * FT];
  alignas(16) float lnb[16 * FT];
};

constexpr int kReadoutWaves = 8;
constexpr int kReadoutTilesPerWave = 2;
constexpr int kReadoutRounds = 2;  // rounds of tiles per wave over one staging of W
constexpr int kReadoutChunk = 16 * kReadoutWaves * kReadoutTilesPerWave * kReadoutRounds;  // tokens per workgroup

template <typename T, int FT, int HTT>
__global__ __launch_bounds__(64 * kReadoutWaves, sizeof(T) == 2 ? 2 : 1) void mlp_readout_kernel(MlpReadoutParams p) {
  constexpr int F = 16 * FT;
  constexpr int FF = 16 * HTT;
  constexpr int NT = kReadoutTilesPerWave;
  __shared__ ReadoutShared<T, FT, HTT> sh;

  // blockIdx -> (chain, chunk): consecutive block ids go to different XCDs, so
  // renumber such that the chunks of a chain sit on the same XCD.
  const int total = gridDim.x;
  int lin = blockIdx.x;
  if ((total & 7) == 0) lin = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int chain = lin / p.nchunk;
  const int chunk = lin - chain * p.nchunk;
  const int h = chain % p.H;

  const int wave = threadIdx.x >> 6;
  const int g = lane_id() >> 4;

  const int ntiles = p.ntok >> 4;
  const size_t xoff = (size_t)chain * p.ntok * F;
  const T* __restrict__ XQ = static_cast<const T*>(p.XQ) + xoff;
  float* __restrict__ OUT = p.out + xoff;

  // XQ^T operand frags of round r (free = token, contraction = feature);
  // tiles past the valid range repeat a valid one and are not stored
  Frag<T> xq[NT][FT];
  auto load_round = [&](int r, int& t0, int& nv) {
    t0 = (chunk * kReadoutRounds + r) * (16 * kReadoutWaves * NT / 16) + wave * NT;  // first token tile
    nv = min(NT, ntiles - t0);                                                    // valid tiles (may be <= 0)
    const int tl = max(nv, 1) - 1;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const T* x = XQ + (size_t)(min(t0 + min(t, tl), ntiles - 1)) * 16 * F;
#pragma unroll
      for (int kb = 0; kb < FT; ++kb) xq[t][kb] = load_frag(x, F, 16 * kb);
    }
  };
  int t0, nv;
  load_round(0, t0, nv);  // requested before the staging

  // ---- stage W1, W2, biases and LN parameters of this chain
  {
    const size_t S = (size_t)p.S;
    stage_fixed_mlp<T, FT, HTT, kReadoutWaves>(sh.w, p.W1 + (size_t)chain * S * F * FF, p.b1 + (size_t)chain * S * FF,
                                               p.W2 + (size_t)chain * S * FF * F, p.b2 + (size_t)chain * S * F);
    for (int i = threadIdx.x; i < F; i += 64 * kReadoutWaves) {
      sh.lnw[i] = p.ln_w[h * F + i];
      sh.lnb[i] = p.ln_b[h * F + i];
    }
  }
  __syncthreads();  // the last barrier: a wave may leave after it

  const float invF = 1.0f / (float)F;
#pragma unroll 1
  for (int r = 0; r < kReadoutRounds; ++r) {
    if (r > 0) load_round(r, t0, nv);
    if (nv <= 0) break;  // later rounds lie further along

    Tile acc[NT][FT];  // Z2 + b2
    fixed_mlp_tiles<T, FT, HTT, NT>(sh.w, xq, acc);

    // ---- LayerNorm over the F features of each token row, residual, store.
    // Lane (g, n) holds 4 features of token n in each feature tile; the row's
    // other 3F/4 features are in lanes n + 16, n + 32, n + 48 (sum_col4).
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t >= nv) break;
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < FT; ++c) s += (acc[t][c].v[0] + acc[t][c].v[1]) + (acc[t][c].v[2] + acc[t][c].v[3]);
      const float mean = sum_col4(s) * invF;
      float q = 0.f;
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        acc[t][c].v -= mean;
        const f4 d = acc[t][c].v;
        q += (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]);
      }
      const float rstd = rsqrt_f(sum_col4(q) * invF + p.eps);
      float* o = OUT + (size_t)(t0 + t) * 16 * F;
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        const f4 lw = *reinterpret_cast<const f4*>(&sh.lnw[16 * c + 4 * g]);
        const f4 lb = *reinterpret_cast<const f4*>(&sh.lnb[16 * c + 4 * g]);
        const f4 x = frag_to_f4(xq[t][c]);  // XQ[n][16c + 4g + j]
        store_f4(o, F, 16 * c, x + lw * (acc[t][c].v * rstd) + lb);
      }
    }
  }
}

template <typename T, int FT, int HTT>
static hipError_t launch_readout_t(const MlpReadoutParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((mlp_readout_kernel<T, FT, HTT>), dim3(p.B * p.H * p.nchunk), dim3(64 * kReadoutWaves), 0,
                     stream, p);
  return hipGetLastError();
}

template <typename T, int FT>
static hipError_t launch_readout_f(const MlpReadoutParams& p, hipStream_t stream) {
  switch (p.FF) {
    case 32: return launch_readout_t<T, FT, 2>(p, stream);
    case 64: return launch_readout_t<T, FT, 4>(p, stream);
    case 128: return launch_readout_t<T, FT, 8>(p, stream);
    case 256: return launch_readout_t<T, FT, 16>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

int mlp_readout_chunk_tokens() { return kReadoutChunk; }

hipError_t launch_mlp_readout(const MlpReadoutParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_readout_f<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_readout_f<__bf16, 2>(p, stream);
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_readout_f<_Float16, 4>(p, stream);
    if (p.F == 32) return launch_readout_f<_Float16, 2>(p, stream);
  } else {
    if (p.F == 64) return launch_readout_f<float, 4>(p, stream);
    if (p.F == 32) return launch_readout_f<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
