// Tile algebra for one wavefront on gfx950 (CDNA4) MFMA.
//
// Every matrix the TTT kernels touch has a 16-row token dimension (one
// mini-batch of K = 16 tokens) or is a fast weight made of 16x16 blocks, so
// all products are built from 16x16 output tiles:
//
//   Tile (fp32 accumulator, "C layout" of v_mfma_f32_16x16x*):
//       lane l = 16*g + n (g = l>>4 in 0..3, n = l&15) holds X[4g + j][n], j = 0..3.
//   Frag<T> (one K16 operand fragment):
//       lane l = 16*g + r holds four values P[r][4g + j], j = 0..3: the lane
//       index r runs over the operand's free index (a row of A, a column of B)
//       and the register index over 4 consecutive contraction indices.
//
// A product Y[m][n] = sum_k P[m][k] Q[k][n] takes P as frags (free = m,
// contraction = k) and Q as frags (free = n, contraction = k).  A C-layout
// tile of X [rows x cols] *is* a frag set with free = cols, contraction = rows
// (the register index runs over rows), so an accumulator can be fed straight
// back into a product that contracts over its rows -- as the right factor X or
// as the left factor X^T.  Contracting over its columns needs a transpose,
// which `transpose16` does exactly with one MFMA against the identity.
//
// A 32-deep contraction step (v_mfma_f32_16x16x32_bf16) packs two K16 frags:
// elements 0-3 carry k-block 2c and elements 4-7 k-block 2c+1.  Any fixed
// permutation of k that is the same for both operands gives the same sum, so
// this packing lets a pair of C-layout tiles (rows 0-15 and 16-31) serve as a
// K32 operand with no data movement.
//
// fp32 activations use v_mfma_f32_16x16x4_f32 (four per K16 frag, register j
// of every lane group in the j-th instruction), which keeps the same frag
// layout and gives fp32-exact products.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ttt_lds_layout.h"

namespace ttt {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

struct Tile {
  f4 v;
};

template <typename T> struct FragT;
template <> struct FragT<float> { typedef f4 type; };
template <> struct FragT<__bf16> { typedef bf4 type; };
template <> struct FragT<_Float16> { typedef h4 type; };

template <typename T> struct Frag {
  typename FragT<T>::type v;
};

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ __bf16 to_bf16(float x) { return (__bf16)x; }

template <typename T> __device__ __forceinline__ Frag<T> to_frag(f4 x);
template <> __device__ __forceinline__ Frag<float> to_frag<float>(f4 x) { return Frag<float>{x}; }
template <> __device__ __forceinline__ Frag<__bf16> to_frag<__bf16>(f4 x) {
  Frag<__bf16> f;
  f.v[0] = (__bf16)x[0];
  f.v[1] = (__bf16)x[1];
  f.v[2] = (__bf16)x[2];
  f.v[3] = (__bf16)x[3];
  return f;
}

// fp32 -> fp16 with the value complete in fp32 registers first.  The empty asm
// keeps the compiler from folding the arithmetic that produced x into the
// conversion (v_fma_mixlo_f16 / v_fma_mixhi_f16 pairs): in the spilled
// K = 64 Linear backward those fused forms gave wrong input gradients from the
// second mini-batch on, while plain conversions (v_cvt_pk_f16_f32) of the same
// values match the fp64 oracle.
__device__ __forceinline__ h4 f16x4_of(f4 x) {
  asm("" : "+v"(x));
  return h4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
}
template <> __device__ __forceinline__ Frag<_Float16> to_frag<_Float16>(f4 x) {
  Frag<_Float16> f;
  f.v = f16x4_of(x);
  return f;
}

template <typename T> __device__ __forceinline__ f4 frag_to_f4(Frag<T> f) {
  return f4{(float)f.v[0], (float)f.v[1], (float)f.v[2], (float)f.v[3]};
}

// exact sign flip of every element
__device__ __forceinline__ Frag<__bf16> negate(Frag<__bf16> f) {
  typedef unsigned short us4 __attribute__((ext_vector_type(4)));
  const us4 m = {0x8000, 0x8000, 0x8000, 0x8000};
  Frag<__bf16> r;
  r.v = __builtin_bit_cast(bf4, __builtin_bit_cast(us4, f.v) ^ m);
  return r;
}
__device__ __forceinline__ Frag<_Float16> negate(Frag<_Float16> f) {
  typedef unsigned short us4 __attribute__((ext_vector_type(4)));
  const us4 m = {0x8000, 0x8000, 0x8000, 0x8000};
  Frag<_Float16> r;
  r.v = __builtin_bit_cast(h4, __builtin_bit_cast(us4, f.v) ^ m);
  return r;
}
__device__ __forceinline__ Frag<float> negate(Frag<float> f) { return Frag<float>{-f.v}; }

// ---------------------------------------------------------------- MFMA
// acc += P * Q over one 16-deep k-block.
//
// bf16 uses only v_mfma_f32_16x16x32_bf16 (upper k-half zero for a 16-deep
// block).  On gfx950, a 16x16x16 bf16 MFMA issued back to back with a
// 16x16x32 bf16 MFMA that reads its result as the accumulator produces wrong
// values unless the pair is padded, and the compiler inserts no padding for
// that mixed-opcode pair; same-opcode accumulation chains are forwarded
// correctly.  Both opcodes issue at the same rate, so the zero half is free.
__device__ __forceinline__ void mma16(f4& acc, Frag<__bf16> p, Frag<__bf16> q) {
  const bf4 z = {(__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f};
  const bf8 a = __builtin_shufflevector(p.v, z, 0, 1, 2, 3, 4, 5, 6, 7);
  const bf8 b = __builtin_shufflevector(q.v, z, 0, 1, 2, 3, 4, 5, 6, 7);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
// fp16 the same way: only v_mfma_f32_16x16x32_f16, the upper k-half zero
__device__ __forceinline__ void mma16(f4& acc, Frag<_Float16> p, Frag<_Float16> q) {
  const h4 z = {(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
  const h8 a = __builtin_shufflevector(p.v, z, 0, 1, 2, 3, 4, 5, 6, 7);
  const h8 b = __builtin_shufflevector(q.v, z, 0, 1, 2, 3, 4, 5, 6, 7);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma16(f4& acc, Frag<float> p, Frag<float> q) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p.v[0], q.v[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p.v[1], q.v[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p.v[2], q.v[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p.v[3], q.v[3], acc, 0, 0, 0);
}
// acc += P * Q over two 16-deep k-blocks (p0/q0 = block 2c, p1/q1 = block 2c+1)
__device__ __forceinline__ void mma32(f4& acc, Frag<__bf16> p0, Frag<__bf16> p1, Frag<__bf16> q0,
                                      Frag<__bf16> q1) {
  bf8 a = __builtin_shufflevector(p0.v, p1.v, 0, 1, 2, 3, 4, 5, 6, 7);
  bf8 b = __builtin_shufflevector(q0.v, q1.v, 0, 1, 2, 3, 4, 5, 6, 7);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma32(f4& acc, Frag<_Float16> p0, Frag<_Float16> p1, Frag<_Float16> q0,
                                      Frag<_Float16> q1) {
  h8 a = __builtin_shufflevector(p0.v, p1.v, 0, 1, 2, 3, 4, 5, 6, 7);
  h8 b = __builtin_shufflevector(q0.v, q1.v, 0, 1, 2, 3, 4, 5, 6, 7);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma32(f4& acc, Frag<float> p0, Frag<float> p1, Frag<float> q0, Frag<float> q1) {
  mma16(acc, p0, q0);
  mma16(acc, p1, q1);
}

// Y[MT x NT tiles] += P (MT free tiles x KB k-blocks) * Q (NT free tiles x KB k-blocks)
template <int MT, int NT, int KB, typename T>
__device__ __forceinline__ void gemm(Tile (&y)[MT][NT], const Frag<T> (&p)[MT][KB], const Frag<T> (&q)[NT][KB]) {
#pragma unroll
  for (int c = 0; c + 1 < KB; c += 2)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < NT; ++n) mma32(y[m][n].v, p[m][c], p[m][c + 1], q[n][c], q[n][c + 1]);
  if (KB & 1) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < NT; ++n) mma16(y[m][n].v, p[m][KB - 1], q[n][KB - 1]);
  }
}

// Y[MT x NT] += P (frags [MT][KB]) * X where X is held as C-layout tiles
// w[KB][NT] of the matrix [16*KB x 16*NT] (contraction over its rows);
// operand frags are converted just before each MFMA.
template <int MT, int NT, int KB, typename T>
__device__ __forceinline__ void gemm_pt(Tile (&y)[MT][NT], const Frag<T> (&p)[MT][KB], const Tile (&w)[KB][NT]) {
#pragma unroll
  for (int n = 0; n < NT; ++n) {
#pragma unroll
    for (int c = 0; c + 1 < KB; c += 2) {
      const Frag<T> q0 = to_frag<T>(w[c][n].v), q1 = to_frag<T>(w[c + 1][n].v);
#pragma unroll
      for (int m = 0; m < MT; ++m) mma32(y[m][n].v, p[m][c], p[m][c + 1], q0, q1);
    }
    if (KB & 1) {
      const Frag<T> q = to_frag<T>(w[KB - 1][n].v);
#pragma unroll
      for (int m = 0; m < MT; ++m) mma16(y[m][n].v, p[m][KB - 1], q);
    }
  }
}
// Y[MT x NT] += X^T * Q with X held as C-layout tiles w[KB][MT] of [16*KB x 16*MT]
template <int MT, int NT, int KB, typename T>
__device__ __forceinline__ void gemm_tp(Tile (&y)[MT][NT], const Tile (&w)[KB][MT], const Frag<T> (&q)[NT][KB]) {
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int c = 0; c + 1 < KB; c += 2) {
      const Frag<T> p0 = to_frag<T>(w[c][m].v), p1 = to_frag<T>(w[c + 1][m].v);
#pragma unroll
      for (int n = 0; n < NT; ++n) mma32(y[m][n].v, p0, p1, q[n][c], q[n][c + 1]);
    }
    if (KB & 1) {
      const Frag<T> p0 = to_frag<T>(w[KB - 1][m].v);
#pragma unroll
      for (int n = 0; n < NT; ++n) mma16(y[m][n].v, p0, q[n][KB - 1]);
    }
  }
}

// The identity as a K16 frag: lane (g, r) holds I[r][4g + j] (symmetric).
template <typename T> __device__ __forceinline__ Frag<T> identity_frag() {
  const int l = lane_id();
  const int g = l >> 4, r = l & 15;
  f4 x;
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = (4 * g + j == r) ? 1.0f : 0.0f;
  return to_frag<T>(x);
}

// Frag P (free = a, contraction = b) -> C-layout tile of the matrix [a x b],
// i.e. a frag with free = b, contraction = a.  Exact: P*I.
template <typename T> __device__ __forceinline__ Tile transpose16(Frag<T> p, Frag<T> ident) {
  Tile t;
  t.v = f4{0.f, 0.f, 0.f, 0.f};
  mma16(t.v, p, ident);
  return t;
}

// Square block of operand frags of X (a[p][q]: free = block p, contraction =
// block q) -> frags of X^T (b[q][p]: free = block q, contraction = block p).
// Exact for values representable in T.
template <int N, typename T>
__device__ __forceinline__ void transpose_frags(const Frag<T> (&a)[N][N], Frag<T> (&b)[N][N], Frag<T> ident) {
#pragma unroll
  for (int p = 0; p < N; ++p)
#pragma unroll
    for (int q = 0; q < N; ++q) b[q][p] = to_frag<T>(transpose16(a[p][q], ident).v);
}

// ---------------------------------------------------------------- lane reductions
template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// sum over the 16 lanes that share g (one DPP row)
__device__ __forceinline__ float sum_row16(float x) {
  x += dpp<0x128>(x);  // row_ror:8
  x += dpp<0x124>(x);  // row_ror:4
  x += dpp<0x122>(x);  // row_ror:2
  x += dpp<0x121>(x);  // row_ror:1
  return x;
}
// max over the 16 lanes that share g (one DPP row)
__device__ __forceinline__ float max_row16(float x) {
  x = fmaxf(x, dpp<0x128>(x));
  x = fmaxf(x, dpp<0x124>(x));
  x = fmaxf(x, dpp<0x122>(x));
  x = fmaxf(x, dpp<0x121>(x));
  return x;
}
// sum over the 4 lanes that share n (lanes n, n+16, n+32, n+48)
// with gfx950's lane swaps (VALU, no trip through the LDS crossbar):
// v_permlane32_swap exchanges the upper half of its first operand with the
// lower half of its second, so with both operands x the two results hold x and
// x^32 in every lane (in either order) and their sum is x + x^32;
// v_permlane16_swap does the same for odd and even 16-lane rows.
__device__ __forceinline__ float sum_col4(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float y = __builtin_bit_cast(float, (unsigned)h[0]) + __builtin_bit_cast(float, (unsigned)h[1]);
  const unsigned v = __builtin_bit_cast(unsigned, y);
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
// sum over all 64 lanes, in every lane: the row sums (sum_row16, equal in
// the 16 lanes of a row) are added across rows with the two lane swaps of
// sum_col4.  Each step adds a pair of lanes that then hold the same sum, so
// every lane ends with the bitwise same value, and nothing goes through a
// scalar register.
__device__ __forceinline__ float sum_wave(float x) { return sum_col4(sum_row16(x)); }
// v[j] summed over all 64 lanes for j = 0..3 at once, in every lane.  The four
// reductions share their steps: the first lane swap of v[0] against v[1]
// (v[2] against v[3]) leaves lanes 0-31 with v[0] (v[2]) and lanes 32-63
// with v[1] (v[3]) summed over lanes l, l^32; the second swap of those two
// against each other leaves 16-lane rows 0..3 with v[0], v[2], v[1], v[3]
// summed over the four lanes l, l^16, l^32, l^48; sum_row16 finishes each row,
// and two more swaps broadcast the four row totals to every lane.  13
// instructions instead of 4 x 8, each result bitwise equal in all lanes.
__device__ __forceinline__ f4 sum4_wave(f4 v) {
  auto bits = [](float x) { return __builtin_bit_cast(unsigned, x); };
  auto flt = [](unsigned x) { return __builtin_bit_cast(float, x); };
  const auto a = __builtin_amdgcn_permlane32_swap(bits(v[0]), bits(v[1]), false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(bits(v[2]), bits(v[3]), false, false);
  const float p = flt((unsigned)a[0]) + flt((unsigned)a[1]);  // lanes < 32: v[0], else v[1]
  const float q = flt((unsigned)b[0]) + flt((unsigned)b[1]);  // lanes < 32: v[2], else v[3]
  const auto c = __builtin_amdgcn_permlane16_swap(bits(p), bits(q), false, false);
  // rows 0, 1, 2, 3: v[0], v[2], v[1], v[3]
  const unsigned r = bits(sum_row16(flt((unsigned)c[0]) + flt((unsigned)c[1])));
  const auto d = __builtin_amdgcn_permlane16_swap(r, r, false, false);  // [0]: v[0] | v[1], [1]: v[2] | v[3]
  const auto e0 = __builtin_amdgcn_permlane32_swap((unsigned)d[0], (unsigned)d[0], false, false);
  const auto e1 = __builtin_amdgcn_permlane32_swap((unsigned)d[1], (unsigned)d[1], false, false);
  return f4{flt((unsigned)e0[0]), flt((unsigned)e0[1]), flt((unsigned)e1[0]), flt((unsigned)e1[1])};
}

// ---------------------------------------------------------------- loads / stores
// Load a K16 frag from a row-major matrix: lane (g, r) reads
// X[r][c0 + 4g .. c0 + 4g + 3] (row stride ld elements).
__device__ __forceinline__ Frag<__bf16> load_frag(const __bf16* __restrict__ x, int ld, int c0) {
  const int l = lane_id();
  const int g = l >> 4, r = l & 15;
  Frag<__bf16> f;
  f.v = *reinterpret_cast<const bf4*>(x + r * ld + c0 + 4 * g);
  return f;
}
__device__ __forceinline__ Frag<_Float16> load_frag(const _Float16* __restrict__ x, int ld, int c0) {
  const int l = lane_id();
  const int g = l >> 4, r = l & 15;
  Frag<_Float16> f;
  f.v = *reinterpret_cast<const h4*>(x + r * ld + c0 + 4 * g);
  return f;
}
__device__ __forceinline__ Frag<float> load_frag(const float* __restrict__ x, int ld, int c0) {
  const int l = lane_id();
  const int g = l >> 4, r = l & 15;
  Frag<float> f;
  f.v = *reinterpret_cast<const f4*>(x + r * ld + c0 + 4 * g);
  return f;
}
// four values X[r][c0 + 4g + j] as fp32 (same pattern, any element type)
template <typename T> __device__ __forceinline__ f4 load_f4(const T* __restrict__ x, int ld, int c0) {
  return frag_to_f4(load_frag(x, ld, c0));
}

// four consecutive values at p as fp32
__device__ __forceinline__ f4 load4(const __bf16* __restrict__ p) {
  const bf4 v = *reinterpret_cast<const bf4*>(p);
  return f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ f4 load4(const _Float16* __restrict__ p) {
  const h4 v = *reinterpret_cast<const h4*>(p);
  return f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ f4 load4(const float* __restrict__ p) { return *reinterpret_cast<const f4*>(p); }
// four consecutive values at p from fp32
__device__ __forceinline__ void store4(__bf16* __restrict__ p, f4 v) {
  *reinterpret_cast<bf4*>(p) = to_frag<__bf16>(v).v;
}
__device__ __forceinline__ void store4(_Float16* __restrict__ p, f4 v) {
  *reinterpret_cast<h4*>(p) = to_frag<_Float16>(v).v;
}
__device__ __forceinline__ void store4(float* __restrict__ p, f4 v) { *reinterpret_cast<f4*>(p) = v; }

// N (2 or 4) consecutive values at p as fp32, one vector access
template <int N> __device__ __forceinline__ void load_n(const float* __restrict__ p, float (&v)[N]) {
  if constexpr (N == 4) {
    const f4 x = *reinterpret_cast<const f4*>(p);
    for (int k = 0; k < 4; ++k) v[k] = x[k];
  } else {
    const f2 x = *reinterpret_cast<const f2*>(p);
    for (int k = 0; k < 2; ++k) v[k] = x[k];
  }
}
template <int N> __device__ __forceinline__ void load_n(const __bf16* __restrict__ p, float (&v)[N]) {
  if constexpr (N == 4) {
    const bf4 x = *reinterpret_cast<const bf4*>(p);
    for (int k = 0; k < 4; ++k) v[k] = (float)x[k];
  } else {
    const bf2 x = *reinterpret_cast<const bf2*>(p);
    for (int k = 0; k < 2; ++k) v[k] = (float)x[k];
  }
}
template <int N> __device__ __forceinline__ void load_n(const _Float16* __restrict__ p, float (&v)[N]) {
  if constexpr (N == 4) {
    const h4 x = *reinterpret_cast<const h4*>(p);
    for (int k = 0; k < 4; ++k) v[k] = (float)x[k];
  } else {
    const h2 x = *reinterpret_cast<const h2*>(p);
    for (int k = 0; k < 2; ++k) v[k] = (float)x[k];
  }
}
template <int N> __device__ __forceinline__ void store_n(float* __restrict__ p, const float (&v)[N]) {
  if constexpr (N == 4) {
    *reinterpret_cast<f4*>(p) = f4{v[0], v[1], v[2], v[3]};
  } else {
    *reinterpret_cast<f2*>(p) = f2{v[0], v[1]};
  }
}
template <int N> __device__ __forceinline__ void store_n(__bf16* __restrict__ p, const float (&v)[N]) {
  if constexpr (N == 4) {
    *reinterpret_cast<bf4*>(p) = bf4{(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
  } else {
    *reinterpret_cast<bf2*>(p) = bf2{(__bf16)v[0], (__bf16)v[1]};
  }
}

template <int N> __device__ __forceinline__ void store_n(_Float16* __restrict__ p, const float (&v)[N]) {
  if constexpr (N == 4) {
    *reinterpret_cast<h4*>(p) = f16x4_of(f4{v[0], v[1], v[2], v[3]});
  } else {
    const h4 h = f16x4_of(f4{v[0], v[1], 0.f, 0.f});
    *reinterpret_cast<h2*>(p) = h2{h[0], h[1]};
  }
}

// Store four values to X[r][c0 + 4g + j]
__device__ __forceinline__ void store_f4(__bf16* __restrict__ x, int ld, int c0, f4 v) {
  const int l = lane_id();
  const int g = l >> 4, r = l & 15;
  *reinterpret_cast<bf4*>(x + r * ld + c0 + 4 * g) = to_frag<__bf16>(v).v;
}
__device__ __forceinline__ void store_f4(_Float16* __restrict__ x, int ld, int c0, f4 v) {
  const int l = lane_id();
  const int g = l >> 4, r = l & 15;
  *reinterpret_cast<h4*>(x + r * ld + c0 + 4 * g) = to_frag<_Float16>(v).v;
}
__device__ __forceinline__ void store_f4(float* __restrict__ x, int ld, int c0, f4 v) {
  const int l = lane_id();
  const int g = l >> 4, r = l & 15;
  *reinterpret_cast<f4*>(x + r * ld + c0 + 4 * g) = v;
}

// C-layout tile <-> row-major fp32 matrix block at (r0, c0)
__device__ __forceinline__ Tile load_tile(const float* __restrict__ x, int ld, int r0, int c0) {
  const int l = lane_id();
  const int g = l >> 4, n = l & 15;
  Tile t;
#pragma unroll
  for (int j = 0; j < 4; ++j) t.v[j] = x[(r0 + 4 * g + j) * ld + c0 + n];
  return t;
}
__device__ __forceinline__ void store_tile(float* __restrict__ x, int ld, int r0, int c0, Tile t) {
  const int l = lane_id();
  const int g = l >> 4, n = l & 15;
#pragma unroll
  for (int j = 0; j < 4; ++j) x[(r0 + 4 * g + j) * ld + c0 + n] = t.v[j];
}

// fp32 matrix [rows][COLS] in LDS as 16 x 16 blocks with a swizzle inside
// each block (lds::blk_elem, csrc/ttt_lds_layout.h): C-layout tiles (lanes of
// group g at rows 4g + j, 16 consecutive columns; four 4-byte accesses) and
// row-vector frags (lanes of group g at 4 consecutive columns of 16 rows; one
// 16-byte access) are both read and written without bank conflicts and with
// no padding.  COLS % 16 == 0; the base is 256-byte aligned.
//
// A view fixes a uniform column offset cw (a multiple of 16).  Every block
// has the same swizzle, so a lane's share of an address does not depend on
// the block: five lane base addresses (the four tile rows j and the row
// vectors) plus the block's constant start r0 * COLS + 16 * c0 (r0, c0
// multiples of 16), which the LDS instruction's 16-bit immediate offset
// absorbs (rows * COLS * 4 <= 64 KB).  `pin()` makes the bases opaque to the
// optimiser; called once per loop iteration it keeps the compiler from
// hoisting every base + constant sum out of the loop into its own register.
typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) f4 lds_f4;

template <int COLS> struct LdsMat {
  static_assert(COLS % 16 == 0, "16 x 16 blocks");
  unsigned tb[4];  // tile lane base addresses of rows j
  unsigned rb;     // row-vector lane base address
  __device__ __forceinline__ LdsMat(float* base, int cw) {
    const unsigned p = (unsigned)(uintptr_t)(lds_f32*)base + 4u * (unsigned)lds::col_base(cw);
    const int l = lane_id(), g = l >> 4, n = l & 15;
#pragma unroll
    for (int j = 0; j < 4; ++j) tb[j] = p + 4u * (unsigned)lds::tile_lane(g, n, j);
    rb = p + 4u * (unsigned)lds::row_lane(g, n);
  }
  __device__ __forceinline__ void pin() {
#pragma unroll
    for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(tb[j]));
    asm volatile("" : "+v"(rb));
  }
  __device__ __forceinline__ static lds_f32* at(unsigned a) { return (lds_f32*)(uintptr_t)a; }
  // C-layout tile at (r0, cw + c0): lane (g, n) holds M[r0 + 4g + j][cw + c0 + n]
  __device__ __forceinline__ Tile tile(int r0, int c0) const {
    const int k = lds::blk_base(COLS, r0, c0);
    Tile t;
#pragma unroll
    for (int j = 0; j < 4; ++j) t.v[j] = at(tb[j])[k];
    return t;
  }
  __device__ __forceinline__ void put_tile(int r0, int c0, Tile t) const {
    const int k = lds::blk_base(COLS, r0, c0);
#pragma unroll
    for (int j = 0; j < 4; ++j) at(tb[j])[k] = t.v[j];
  }
  // row-vector frag at (r0, cw + c0): lane (g, r) holds M[r0 + r][cw + c0 + 4g + j]
  __device__ __forceinline__ f4 row4(int r0, int c0) const {
    return *reinterpret_cast<lds_f4*>(at(rb) + lds::blk_base(COLS, r0, c0));
  }
  __device__ __forceinline__ void put_row4(int r0, int c0, f4 v) const {
    *reinterpret_cast<lds_f4*>(at(rb) + lds::blk_base(COLS, r0, c0)) = v;
  }
};

// One lane's 16-byte slot in an LDS region laid out in lane order ([...][64]
// x 16 bytes): the lane's address is a single register and every block of the
// region a compile-time immediate offset (< 64 KB).  `pin()` as for LdsMat.
struct LdsLane {
  unsigned a;
  __device__ __forceinline__ LdsLane(void* base, int byte_off) {
    a = (unsigned)(uintptr_t)(lds_f32*)base + (unsigned)byte_off + 16u * (unsigned)lane_id();
  }
  __device__ __forceinline__ void pin() { asm volatile("" : "+v"(a)); }
  __device__ __forceinline__ f4 get(int off) const { return *reinterpret_cast<lds_f4*>((lds_f32*)(uintptr_t)a + off / 4); }
  __device__ __forceinline__ void put(int off, f4 v) const {
    *reinterpret_cast<lds_f4*>((lds_f32*)(uintptr_t)a + off / 4) = v;
  }
};

// Tile registers <-> scratch in register order (fully coalesced float4 per lane)
__device__ __forceinline__ void spill_tile(float* __restrict__ x, Tile t) {
  reinterpret_cast<f4*>(x)[lane_id()] = t.v;
}
__device__ __forceinline__ Tile fill_tile(const float* __restrict__ x) {
  Tile t;
  t.v = reinterpret_cast<const f4*>(x)[lane_id()];
  return t;
}

// ---------------------------------------------------------------- fast reciprocals
// v_rcp_f32 / v_rsq_f32 (about 1 ulp) instead of the IEEE divide and square
// root sequences; every argument here is a normal positive number.
__device__ __forceinline__ float rcp_f(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float rsqrt_f(float x) { return __builtin_amdgcn_rsqf(x); }

// ---------------------------------------------------------------- GELU (tanh form)
// F.gelu(x, approximate="tanh") = 0.5 x (1 + tanh(u)), u = k x (1 + c x^2),
// rewritten with 0.5 (1 + tanh(u)) = sigma(2u) = 1 / (1 + 2^(-2 log2(e) u)):
// one v_exp_f32 and one v_rcp_f32, no cancellation in 1 + tanh for negative
// x, and the right limits (2^(+big) = inf gives sigma = 0, 2^(-big) = 0 gives
// sigma = 1).  With s = sigma(2u), q = s (1 - s) and D = du/dx = k + 3 c k x^2:
//   gelu    = x s
//   gelu'   = s + 2 x q D                          (ops/ttt_utils.py:51-54)
//   gelu''  = 4 q (D + x (1 - 2 s) D^2 + 3 c k x^2)
// the derivatives of 0.5 x (1 + tanh u) written in s (tanh u = 2 s - 1,
// 1 - tanh^2 u = 4 q).
constexpr float kGeluK = 0.7978845608028654f;                     // sqrt(2 / pi)
constexpr float kGeluC = 0.044715f;
constexpr float kGeluC3 = 3.0f * kGeluC * kGeluK;                  // 0.1070322243
constexpr float kGeluA = -2.0f * 1.4426950408889634f * kGeluK;     // -2 log2(e) k
constexpr float kGeluB = kGeluA * kGeluC;

// sigma(2u) given x and x^2
__device__ __forceinline__ float gelu_sig(float x, float x2) {
  return rcp_f(1.0f + __builtin_amdgcn_exp2f(x * __builtin_fmaf(kGeluB, x2, kGeluA)));
}
__device__ __forceinline__ float gelu_tanh(float x) { return x * gelu_sig(x, x * x); }
// gelu(x) and gelu'(x)
__device__ __forceinline__ void gelu_fwd_bwd(float x, float& y, float& dy) {
  const float x2 = x * x;
  const float s = gelu_sig(x, x2);
  const float D = __builtin_fmaf(kGeluC3, x2, kGeluK);
  y = x * s;
  dy = __builtin_fmaf(2.0f * x * D, s - s * s, s);
}
// gelu(x), gelu'(x) and gelu''(x)
__device__ __forceinline__ void gelu_all(float x, float& y, float& dy, float& ddy) {
  const float x2 = x * x;
  const float s = gelu_sig(x, x2);
  const float D = __builtin_fmaf(kGeluC3, x2, kGeluK);
  const float q = s - s * s;
  const float xD = x * D;
  y = x * s;
  dy = __builtin_fmaf(2.0f * xD, q, s);
  ddy = 4.0f * q * (D + __builtin_fmaf(kGeluC3, x2, xD * D * (1.0f - 2.0f * s)));
}

}  // namespace ttt
