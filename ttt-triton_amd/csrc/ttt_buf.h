// Buffer (MUBUF) access for the per-chain slabs the kernels stream.
//
// A buffer resource (4 SGPRs) holds a slab's base and byte size; every access
// is resource + 32-bit lane offset (one VGPR shared by all slabs with the same
// layout) + uniform offset (SGPR) + immediate.  Compared with 64-bit flat
// addresses this keeps one VGPR per access pattern instead of a VGPR pair per
// pointer, and accesses past the slab's end read 0 / write nothing.
#pragma once

#include "ttt_tile.h"

namespace ttt {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned int u2v __attribute__((ext_vector_type(2)));
typedef unsigned int u4v __attribute__((ext_vector_type(4)));

// gfx9-family buffer descriptor word 3 (raw, untyped 32-bit access)
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, unsigned int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufferWord3);
}

// A lane offset that the range check drops when `keep` is false: offsets of
// 2^31 and more lie past every slab these kernels address (each is checked to
// stay below 2^31 bytes).  Stores that only some waves or lanes should make go
// through this instead of a branch, so that every wave issues the same memory
// operations and the compiler's wait counts for earlier loads stay exact.
__device__ __forceinline__ int keep_or_drop(int voff, bool keep) {
  return (int)((unsigned)voff | (keep ? 0u : 0x80000000u));
}

// four consecutive elements at byte offset voff + soff
template <typename T> __device__ __forceinline__ Frag<T> bload_frag(rsrc_t r, int voff, int soff);
template <> __device__ __forceinline__ Frag<__bf16> bload_frag<__bf16>(rsrc_t r, int voff, int soff) {
  Frag<__bf16> f;
  f.v = __builtin_bit_cast(bf4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  return f;
}
template <> __device__ __forceinline__ Frag<_Float16> bload_frag<_Float16>(rsrc_t r, int voff, int soff) {
  Frag<_Float16> f;
  f.v = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  return f;
}
template <> __device__ __forceinline__ Frag<float> bload_frag<float>(rsrc_t r, int voff, int soff) {
  Frag<float> f;
  f.v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  return f;
}

template <typename T> __device__ __forceinline__ void bstore_frag(rsrc_t r, int voff, int soff, Frag<T> f);
template <> __device__ __forceinline__ void bstore_frag<__bf16>(rsrc_t r, int voff, int soff, Frag<__bf16> f) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, f.v), r, voff, soff, 0);
}
template <> __device__ __forceinline__ void bstore_frag<_Float16>(rsrc_t r, int voff, int soff, Frag<_Float16> f) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, f.v), r, voff, soff, 0);
}
template <> __device__ __forceinline__ void bstore_frag<float>(rsrc_t r, int voff, int soff, Frag<float> f) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, f.v), r, voff, soff, 0);
}

// Device-coherent stores (cache policy sc1): written through to memory, so a
// workgroup on another XCD that sees a later flag reads them without an L2
// writeback by the writer.
constexpr int kCpolDevice = 16;  // sc1
template <typename T> __device__ __forceinline__ void bstore_frag_dev(rsrc_t r, int voff, int soff, Frag<T> f);
template <> __device__ __forceinline__ void bstore_frag_dev<__bf16>(rsrc_t r, int voff, int soff, Frag<__bf16> f) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, f.v), r, voff, soff, kCpolDevice);
}
template <> __device__ __forceinline__ void bstore_frag_dev<_Float16>(rsrc_t r, int voff, int soff, Frag<_Float16> f) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, f.v), r, voff, soff, kCpolDevice);
}
template <> __device__ __forceinline__ void bstore_frag_dev<float>(rsrc_t r, int voff, int soff, Frag<float> f) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, f.v), r, voff, soff, kCpolDevice);
}

// Device-coherent loads (sc1): not served from a cache line that another
// XCD's writes may have made stale.
template <typename T> __device__ __forceinline__ Frag<T> bload_frag_dev(rsrc_t r, int voff, int soff);
template <> __device__ __forceinline__ Frag<__bf16> bload_frag_dev<__bf16>(rsrc_t r, int voff, int soff) {
  Frag<__bf16> f;
  f.v = __builtin_bit_cast(bf4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kCpolDevice));
  return f;
}
template <> __device__ __forceinline__ Frag<_Float16> bload_frag_dev<_Float16>(rsrc_t r, int voff, int soff) {
  Frag<_Float16> f;
  f.v = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kCpolDevice));
  return f;
}
template <> __device__ __forceinline__ Frag<float> bload_frag_dev<float>(rsrc_t r, int voff, int soff) {
  Frag<float> f;
  f.v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kCpolDevice));
  return f;
}

// one element, as float
template <typename T> __device__ __forceinline__ float bload1(rsrc_t r, int voff, int soff);
template <> __device__ __forceinline__ float bload1<__bf16>(rsrc_t r, int voff, int soff) {
  const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
  return (float)__builtin_bit_cast(__bf16, u);
}
template <> __device__ __forceinline__ float bload1<_Float16>(rsrc_t r, int voff, int soff) {
  const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
  return (float)__builtin_bit_cast(_Float16, u);
}
template <> __device__ __forceinline__ float bload1<float>(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

__device__ __forceinline__ float bload_f32(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void bstore_f32(rsrc_t r, int voff, int soff, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, voff, soff, 0);
}

// C-layout tile of a row-major fp32 matrix (row stride ld elements) at
// (r0, c0): lane (g, n) reads rows r0 + 4g + j, column c0 + n.  `lane` =
// ((4g) * ld + n) * 4 plus any per-wave column offset; the rest is uniform.
__device__ __forceinline__ Tile bload_tile(rsrc_t r, int lane, int soff, int ld, int r0, int c0) {
  Tile t;
#pragma unroll
  for (int j = 0; j < 4; ++j) t.v[j] = bload_f32(r, lane, soff + ((r0 + j) * ld + c0) * 4);
  return t;
}
__device__ __forceinline__ void bstore_tile(rsrc_t r, int lane, int soff, int ld, int r0, int c0, Tile t) {
#pragma unroll
  for (int j = 0; j < 4; ++j) bstore_f32(r, lane, soff + ((r0 + j) * ld + c0) * 4, t.v[j]);
}

// C-layout tile of a row-major [16 x ld] block in the activation type: lane
// (g, n) gets rows 4g + j, column n (four element loads).  `voff` =
// ((4g) * ld + n) * sizeof(T) plus any column offset; the rest is uniform.
template <typename T> __device__ __forceinline__ Frag<T> bload_ctile(rsrc_t r, int voff, int soff, int ld);
template <> __device__ __forceinline__ Frag<__bf16> bload_ctile<__bf16>(rsrc_t r, int voff, int soff, int ld) {
  typedef unsigned short us4 __attribute__((ext_vector_type(4)));
  us4 u;
#pragma unroll
  for (int j = 0; j < 4; ++j) u[j] = __builtin_amdgcn_raw_buffer_load_b16(r, voff + j * ld * 2, soff, 0);
  Frag<__bf16> f;
  f.v = __builtin_bit_cast(bf4, u);
  return f;
}
template <> __device__ __forceinline__ Frag<_Float16> bload_ctile<_Float16>(rsrc_t r, int voff, int soff, int ld) {
  typedef unsigned short us4 __attribute__((ext_vector_type(4)));
  us4 u;
#pragma unroll
  for (int j = 0; j < 4; ++j) u[j] = __builtin_amdgcn_raw_buffer_load_b16(r, voff + j * ld * 2, soff, 0);
  Frag<_Float16> f;
  f.v = __builtin_bit_cast(h4, u);
  return f;
}
template <> __device__ __forceinline__ Frag<float> bload_ctile<float>(rsrc_t r, int voff, int soff, int ld) {
  Frag<float> f;
#pragma unroll
  for (int j = 0; j < 4; ++j) f.v[j] = bload_f32(r, voff + j * ld * 4, soff);
  return f;
}
template <typename T> __device__ __forceinline__ void bstore_ctile(rsrc_t r, int voff, int soff, int ld, Frag<T> f);
template <> __device__ __forceinline__ void bstore_ctile<__bf16>(rsrc_t r, int voff, int soff, int ld, Frag<__bf16> f) {
  typedef unsigned short us4 __attribute__((ext_vector_type(4)));
  const us4 u = __builtin_bit_cast(us4, f.v);
#pragma unroll
  for (int j = 0; j < 4; ++j) __builtin_amdgcn_raw_buffer_store_b16(u[j], r, voff + j * ld * 2, soff, 0);
}
template <> __device__ __forceinline__ void bstore_ctile<_Float16>(rsrc_t r, int voff, int soff, int ld, Frag<_Float16> f) {
  typedef unsigned short us4 __attribute__((ext_vector_type(4)));
  const us4 u = __builtin_bit_cast(us4, f.v);
#pragma unroll
  for (int j = 0; j < 4; ++j) __builtin_amdgcn_raw_buffer_store_b16(u[j], r, voff + j * ld * 2, soff, 0);
}
template <> __device__ __forceinline__ void bstore_ctile<float>(rsrc_t r, int voff, int soff, int ld, Frag<float> f) {
#pragma unroll
  for (int j = 0; j < 4; ++j) bstore_f32(r, voff + j * ld * 4, soff, f.v[j]);
}

}  // namespace ttt
