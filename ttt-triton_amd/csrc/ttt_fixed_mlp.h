// Fixed-weight two-layer MLP over token tiles, shared by the cached readout
// and the memory-cache combiner:
//
//   Z2 = gelu(X W1 + b1) W2 + b2        X: 16-token tiles, W1 [F x FF], W2 [FF x F]
//
// W1 and W2 sit in LDS in MFMA operand order: the two K16 blocks that form
// one 32-deep operand are stored as consecutive 64-lane blocks, so the operand
// is one ds_read2st64 (two contiguous wave-wide reads, conflict-free) into
// consecutive registers.  The hidden dimension is walked two 16-unit tiles at
// a time:
//
//   Z1^T(pair) = W1^T X^T + b1      hidden x token (C layout = the B operand of
//   X2^T       = gelu(Z1^T)          the next product, no transpose)
//   Z2^T      += W2(pair)^T X2^T     feature x token
//
// Z2 comes out transposed, token-major: the C layout of Z2^T puts one token on
// each lane's free index and four consecutive features in its registers, the
// layout of X's own operand frags and of a 16-byte row store, so the callers'
// per-token LayerNorm needs no transpose and reduces over four lanes only.
//
// (Issuing the next pair's Z1 products ahead of the current GELU was measured
// no faster at B16 H12 T2048 F64 FF256 and costs 16 registers.)
#pragma once

#include "ttt_tile.h"

namespace ttt {

template <typename T, int FT, int HTT> struct FixedMlpLds {
  using V = typename FragT<T>::type;
  V w1[HTT][FT / 2][2][64];  // [ht][kp][h]: W1 block (2kp + h, ht) = W1[16kb + 4g + j][16ht + n]
  V w2[HTT / 2][FT][2][64];  // [hp][ct][h]: W2 block (2hp + h, ct) = W2[16ht + 4g + j][16ct + n]
  alignas(16) float b1[16 * HTT];
  alignas(16) float b2[16 * FT];
};

// Stage one (W1, b1, W2, b2) into LDS with NWAVES waves: each wave takes
// blocks wave, wave + NWAVES, ... of W1 and of W2 and issues every global load
// before the first conversion (bf16; fp32 operands go one matrix at a time to
// bound the registers).  The caller brackets it with barriers.
template <typename T, int FT, int HTT, int NWAVES>
__device__ __forceinline__ void stage_fixed_mlp(FixedMlpLds<T, FT, HTT>& sh, const float* __restrict__ w1,
                                                const float* __restrict__ b1, const float* __restrict__ w2,
                                                const float* __restrict__ b2) {
  constexpr int F = 16 * FT, FF = 16 * HTT, NBLK = FT * HTT;
  constexpr int NB = (NBLK + NWAVES - 1) / NWAVES;
  static_assert(FF <= 64 * NWAVES && F <= 64 * NWAVES, "one bias value per thread");
  const int wave = threadIdx.x >> 6;
  const int l = lane_id(), g = l >> 4, n = l & 15;
  const float bias1 = threadIdx.x < FF ? b1[threadIdx.x] : 0.f;
  const float bias2 = threadIdx.x < F ? b2[threadIdx.x] : 0.f;
  auto load_w1 = [&](f4(&x)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int blk = min(wave + NWAVES * b, NBLK - 1), kb = blk / HTT, ht = blk - kb * HTT;
#pragma unroll
      for (int j = 0; j < 4; ++j) x[b][j] = w1[(16 * kb + 4 * g + j) * FF + 16 * ht + n];
    }
  };
  auto load_w2 = [&](f4(&x)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int blk = min(wave + NWAVES * b, NBLK - 1), ht = blk / FT, ct = blk - ht * FT;
#pragma unroll
      for (int j = 0; j < 4; ++j) x[b][j] = w2[(16 * ht + 4 * g + j) * F + 16 * ct + n];
    }
  };
  auto put_w1 = [&](const f4(&x)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int blk = wave + NWAVES * b, kb = blk / HTT, ht = blk - kb * HTT;
      if (blk < NBLK) sh.w1[ht][kb >> 1][kb & 1][l] = to_frag<T>(x[b]).v;  // (uniform over the wave)
    }
  };
  auto put_w2 = [&](const f4(&x)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int blk = wave + NWAVES * b, ht = blk / FT, ct = blk - ht * FT;
      if (blk < NBLK) sh.w2[ht >> 1][ct][ht & 1][l] = to_frag<T>(x[b]).v;
    }
  };
  if constexpr (sizeof(T) == 2) {
    f4 x1[NB], x2[NB];
    load_w1(x1);
    load_w2(x2);
    put_w1(x1);
    put_w2(x2);
  } else {
    f4 x[NB];
    load_w1(x);
    put_w1(x);
    load_w2(x);
    put_w2(x);
  }
  if (threadIdx.x < FF) sh.b1[threadIdx.x] = bias1;
  if (threadIdx.x < F) sh.b2[threadIdx.x] = bias2;
}

// acc[t][c] = Z2 of token tile t, feature tile c, token-major (lane (g, n)
// holds Z2[n][16c + 4g + j], the C layout of Z2^T), from the operand frags
// xq[t][kb] of X^T (free = token, contraction = feature; lane (g, n) holds
// X[n][16kb + 4g + j]).  b2 is added.
template <typename T, int FT, int HTT, int NT>
__device__ __forceinline__ void fixed_mlp_tiles(const FixedMlpLds<T, FT, HTT>& sh, const Frag<T> (&xq)[NT][FT],
                                                Tile (&acc)[NT][FT]) {
  static_assert(FT % 2 == 0 && HTT % 2 == 0, "pairs of 16-wide tiles");
  const int l = lane_id(), g = l >> 4;
#pragma unroll
  for (int c = 0; c < FT; ++c) {
    const f4 b2 = *reinterpret_cast<const f4*>(&sh.b2[16 * c + 4 * g]);
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][c].v = b2;
  }
  // Z1^T of hidden tiles (ht, ht + 1) for every token tile, b1 in the accumulator
  auto z1 = [&](int ht, Tile (&z)[2][NT]) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      Frag<T> w[FT];
#pragma unroll
      for (int kp = 0; kp < FT / 2; ++kp) {
        w[2 * kp].v = sh.w1[ht + hh][kp][0][l];
        w[2 * kp + 1].v = sh.w1[ht + hh][kp][1][l];
      }
      const f4 bias = *reinterpret_cast<const f4*>(&sh.b1[16 * (ht + hh) + 4 * g]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        z[hh][t].v = bias;
#pragma unroll
        for (int kb = 0; kb < FT; kb += 2) mma32(z[hh][t].v, w[kb], w[kb + 1], xq[t][kb], xq[t][kb + 1]);
      }
    }
  };
#pragma unroll 1
  for (int ht = 0; ht < HTT; ht += 2) {
    Tile z[2][NT];
    z1(ht, z);
    Frag<T> x2[2][NT];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f4 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = gelu_tanh(z[hh][t].v[j]);
        x2[hh][t] = to_frag<T>(a);
      }
#pragma unroll
    for (int c = 0; c < FT; ++c) {
      Frag<T> q0, q1;
      q0.v = sh.w2[ht >> 1][c][0][l];
      q1.v = sh.w2[ht >> 1][c][1][l];
#pragma unroll
      for (int t = 0; t < NT; ++t) mma32(acc[t][c].v, q0, q1, x2[0][t], x2[1][t]);
    }
  }
}

}  // namespace ttt
