// The producer and consumer around the TTT inner loop on gfx950: what
// TTTBase.process_input does between the QKVU projections and the inner
// loop, and what TTTBase.forward does between the inner loop and `wo`.
//
// Producer (ttt_layer.py:261-309), per token row (b, t) and head h of the
// fused projection row proj[b, t] = [XQ | XK | XV | XU | lr logits]:
//   XQ, XK, XU  L2-normalised over the head dim (x / max(|x|, 1e-12),
//               ttt_layer.py:279-281), then rotated by RoPE at position t
//               (utils.py:97-123: pairs (2p, 2p+1) times cos + i sin of the
//               table row t, ttt_layer.py:287-300)
//   XV          the reconstruction target ln_w (d - mean d) / (std d + eps)
//               + ln_b + XK with d = XV - XK and the unbiased std
//               (ttt_layer.py:227-243, eps 1e-8 there)
//   lr          base_lr * sigmoid(logit) / F (ttt_layer.py:151-163)
// written straight into the inner loop's layouts [B,H,NC,K,F] and [B,H,NC,K]
// (ttt_layer.py:245-259), so no permute or copy runs between the two.  The
// backward recomputes the forward from the projection row (everything is
// elementwise or a reduction over one head's F features) and writes the
// gradient of the projection row; the LayerNorm-parameter gradients of the
// target come out as per-block partials.
//
// Consumer (ttt_layer.py:349, 563-564): the inner loop's output [B,H,NC,K,F]
// read per token row as the [H*F] vector the caller's permute + reshape
// gives, LayerNorm over it (post_norm, biased variance, eps 1e-6 there),
// stored as [B, L, H*F]; its backward scatters the gradient back into
// [B,H,NC,K,F].
//
// All four kernels are HBM-bound elementwise passes: one wavefront per token
// row, each lane 4 consecutive features (one 8- or 16-byte access per tensor),
// a head's F features on F/4 lanes, reductions over them by lane swizzles.
#include <math.h>

#include "ttt_kernels.h"

namespace ttt {

namespace {

constexpr int kRowsPerBlockBwd = 16;  // token rows per workgroup in the backwards (LN-parameter partials)
constexpr int kMaxD = 1024;           // H * F

// sum over groups of W consecutive lanes (W = 8 or 16), every lane of a group
// receives its group's sum
template <int W> __device__ __forceinline__ float group_sum(float x) {
  if constexpr (W == 16) {
    return sum_row16(x);
  } else {
    static_assert(W == 8, "group width");
    // ds_swizzle bit mode: lane ^= m within 32-lane halves
    x += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), (4 << 10) | 0x1F));
    x += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), (2 << 10) | 0x1F));
    x += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), (1 << 10) | 0x1F));
    return x;
  }
}

__device__ __forceinline__ float hsum(f4 v) { return (v[0] + v[1]) + (v[2] + v[3]); }
__device__ __forceinline__ f4 splat(float x) { return f4{x, x, x, x}; }

template <typename T> __device__ __forceinline__ f4 ld4(const T* p, bool act) {
  return act ? load4(p) : splat(0.f);
}

// pairs (v0, v1) and (v2, v3) rotated by the angles whose cos/sin are
// cs = (cos_a, sin_a, cos_b, sin_b); `inv` rotates backwards (the transpose)
__device__ __forceinline__ f4 rotate(f4 v, f4 cs, bool inv) {
  const float sa = inv ? -cs[1] : cs[1], sb = inv ? -cs[3] : cs[3];
  f4 r;
  r[0] = v[0] * cs[0] - v[1] * sa;
  r[1] = v[0] * sa + v[1] * cs[0];
  r[2] = v[2] * cs[2] - v[3] * sb;
  r[3] = v[2] * sb + v[3] * cs[2];
  return r;
}

// the forward of one (row, head) share of a lane, everything the backward
// needs as well
template <int F> struct ProducerRow {
  static constexpr int W = F / 4;  // lanes per head
  f4 q, k, u;                      // raw projections
  f4 qn, kn, un;                   // L2-normalised
  float dq, dk, du;                // max(|x|, eps)
  float iq, ik, iu;                // their reciprocals
  f4 qr, kr, ur;                   // rotated
  f4 c;                            // d - mean(d), d = XV - XK_rotated
  float sd;                        // unbiased std of d
  f4 xv;                           // reconstruction target

  __device__ __forceinline__ void run(f4 q_, f4 k_, f4 v, f4 u_, f4 cs, f4 lw, f4 lb, float l2eps, float eps) {
    q = q_;
    k = k_;
    u = u_;
    dq = fmaxf(sqrtf(group_sum<W>(hsum(q * q))), l2eps);
    dk = fmaxf(sqrtf(group_sum<W>(hsum(k * k))), l2eps);
    du = fmaxf(sqrtf(group_sum<W>(hsum(u * u))), l2eps);
    iq = 1.0f / dq;
    ik = 1.0f / dk;
    iu = 1.0f / du;
    qn = q * iq;
    kn = k * ik;
    un = u * iu;
    qr = rotate(qn, cs, false);
    kr = rotate(kn, cs, false);
    ur = rotate(un, cs, false);
    const f4 d = v - kr;
    const float mean = group_sum<W>(hsum(d)) / (float)F;
    c = d - splat(mean);
    sd = sqrtf(group_sum<W>(hsum(c * c)) / (float)(F - 1));
    xv = lw * (c * (1.0f / (sd + eps))) + lb + kr;
  }
};

}  // namespace

template <typename T, int F>
__global__ __launch_bounds__(256) void qkvu_producer_fwd_kernel(ProducerParams p) {
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const long long rows = (long long)p.B * p.L;
  const long long row = (long long)blockIdx.x * 4 + wave;  // b * L + t
  if (row >= rows) return;  // uniform per wave
  const int b = (int)(row / p.L), t = (int)(row - (long long)b * p.L);
  const int D = p.H * F;
  const T* __restrict__ pr = static_cast<const T*>(p.proj) + row * p.ld;
  for (int c0 = 0; c0 < D; c0 += 256) {
    const int c = c0 + 4 * l;
    const bool act = c < D;  // whole heads: D is a multiple of F
    const int h = c / F, f = c - h * F;
    const f4 cs = act ? *reinterpret_cast<const f4*>(p.rope + ((size_t)t * (F / 2) + f / 2) * 2) : splat(0.f);
    const f4 lw = act ? *reinterpret_cast<const f4*>(p.ln_w + h * F + f) : splat(0.f);
    const f4 lb = act ? *reinterpret_cast<const f4*>(p.ln_b + h * F + f) : splat(0.f);
    ProducerRow<F> r;
    r.run(ld4(pr + c, act), ld4(pr + D + c, act), ld4(pr + 2 * D + c, act), ld4(pr + 3 * D + c, act), cs, lw, lb,
          p.l2eps, p.eps);
    if (act) {
      const size_t o = (((size_t)b * p.H + h) * p.L + t) * F + f;
      store4(static_cast<T*>(p.XQ) + o, r.qr);
      store4(static_cast<T*>(p.XK) + o, r.kr);
      store4(static_cast<T*>(p.XV) + o, r.xv);
      store4(static_cast<T*>(p.XU) + o, r.ur);
      if (f == 0) {
        const float z = (float)pr[4 * D + h];
        p.lr[((size_t)b * p.H + h) * p.L + t] = p.base_lr * (1.0f / (1.0f + expf(-z))) / (float)F;
      }
    }
  }
}

template <typename T, int F, int NCH>
__global__ __launch_bounds__(256) void qkvu_producer_bwd_kernel(ProducerParams p) {
  constexpr int W = F / 4;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const long long rows = (long long)p.B * p.L;
  const int D = p.H * F;
  __shared__ float red[4][2][256 * NCH];
  f4 aw[NCH], ab[NCH];  // LN-parameter gradient partials per 256-feature chunk
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    aw[i] = splat(0.f);
    ab[i] = splat(0.f);
  }
  const long long r0 = (long long)blockIdx.x * kRowsPerBlockBwd;
  for (long long row = r0 + wave; row < r0 + kRowsPerBlockBwd && row < rows; row += 4) {
    const int b = (int)(row / p.L), t = (int)(row - (long long)b * p.L);
    const T* __restrict__ pr = static_cast<const T*>(p.proj) + row * p.ld;
    T* __restrict__ dpr = static_cast<T*>(p.dproj) + row * p.ld;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = 256 * i + 4 * l;
      if (256 * i >= D) break;  // uniform
      const bool act = c < D;
      const int h = c / F, f = c - h * F;
      const f4 cs = act ? *reinterpret_cast<const f4*>(p.rope + ((size_t)t * (F / 2) + f / 2) * 2) : splat(0.f);
      const f4 lw = act ? *reinterpret_cast<const f4*>(p.ln_w + h * F + f) : splat(0.f);
      const f4 lb = act ? *reinterpret_cast<const f4*>(p.ln_b + h * F + f) : splat(0.f);
      ProducerRow<F> r;
      r.run(ld4(pr + c, act), ld4(pr + D + c, act), ld4(pr + 2 * D + c, act), ld4(pr + 3 * D + c, act), cs, lw, lb,
            p.l2eps, p.eps);
      const size_t o = (((size_t)b * p.H + h) * p.L + t) * F + f;
      const f4 gq = ld4(static_cast<const T*>(p.dXQ) + o, act);
      const f4 gk = ld4(static_cast<const T*>(p.dXK) + o, act);
      const f4 gv = ld4(static_cast<const T*>(p.dXV) + o, act);
      const f4 gu = ld4(static_cast<const T*>(p.dXU) + o, act);
      // reconstruction target: xv = lw * c / (sd + eps) + lb + kr
      const float den = r.sd + p.eps, iden = 1.0f / den;
      const f4 xhat = r.c * iden;
      aw[i] += gv * xhat;
      ab[i] += gv;
      const f4 y = gv * lw;  // gradient wrt xhat
      const float ymean = group_sum<W>(hsum(y)) / (float)F;
      const float yc = group_sum<W>(hsum(y * r.c));
      // d xhat_i / d d_j = (delta_ij - 1/F) / den - c_i c_j / (den^2 sd (F - 1))
      const float k2 = r.sd > 0.f ? yc / (den * den * r.sd * (float)(F - 1)) : 0.f;
      const f4 dd = (y - splat(ymean)) * iden - r.c * k2;
      const f4 gkr = gk + gv - dd;  // XK enters the target directly and through d = XV - XK
      // rotations back, then the L2 normalisations: d(x / n) = (g - xn (xn . g)) / n where
      // |x| > eps, g / eps elsewhere (n = max(|x|, eps) > eps exactly when |x| > eps)
      const f4 gqn = rotate(gq, cs, true), gkn = rotate(gkr, cs, true), gun = rotate(gu, cs, true);
      auto l2back = [&](f4 xn, f4 g, float n, float in) {
        if (n > p.l2eps) {
          const float dot = group_sum<W>(hsum(xn * g));
          return (g - xn * dot) * in;
        }
        return g * in;
      };
      const f4 dq = l2back(r.qn, gqn, r.dq, r.iq);
      const f4 dk = l2back(r.kn, gkn, r.dk, r.ik);
      const f4 du = l2back(r.un, gun, r.du, r.iu);
      if (act) {
        store4(dpr + c, dq);
        store4(dpr + D + c, dk);
        store4(dpr + 2 * D + c, dd);
        store4(dpr + 3 * D + c, du);
        if (f == 0) {
          const float z = (float)pr[4 * D + h];
          const float sg = 1.0f / (1.0f + expf(-z));
          const float g = p.dlr ? p.dlr[((size_t)b * p.H + h) * p.L + t] : 0.f;
          dpr[4 * D + h] = (T)(g * p.base_lr / (float)F * sg * (1.0f - sg));
        }
      }
    }
    // padding columns of the row (a caller may pad the logits to an aligned width)
    for (int c = 4 * D + p.H + l; c < p.ld; c += 64) dpr[c] = (T)0.0f;
  }
  // per-block LN-parameter partials: waves in fixed order (deterministic)
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = 256 * i + 4 * l;
    if (c < D) {
      *reinterpret_cast<f4*>(&red[wave][0][c]) = aw[i];
      *reinterpret_cast<f4*>(&red[wave][1][c]) = ab[i];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < 2 * D; c += 256) {
    const int k = c / D, j = c - k * D;
    p.partial[((size_t)blockIdx.x * 2 + k) * D + j] = ((red[0][k][j] + red[1][k][j]) + red[2][k][j]) + red[3][k][j];
  }
}

template <typename T, int F>
__global__ __launch_bounds__(256) void post_norm_fwd_kernel(PostNormParams p) {
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const long long rows = (long long)p.B * p.L;
  const long long row = (long long)blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const int b = (int)(row / p.L), t = (int)(row - (long long)b * p.L);
  const int D = p.H * F;
  f4 x[kMaxD / 256];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxD / 256; ++i) {
    const int c = 256 * i + 4 * l;
    const bool act = c < D;
    const int h = c / F, f = c - h * F;
    x[i] = ld4(static_cast<const T*>(p.X) + (((size_t)b * p.H + h) * p.L + t) * F + f, act);
    s += hsum(x[i]);
  }
  const float mean = sum_wave(s) / (float)D;
  float v = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxD / 256; ++i) {
    const int c = 256 * i + 4 * l;
    if (c < D) {
      const f4 d = x[i] - splat(mean);
      v += hsum(d * d);
    }
  }
  const float rstd = 1.0f / sqrtf(sum_wave(v) / (float)D + p.eps);
#pragma unroll
  for (int i = 0; i < kMaxD / 256; ++i) {
    const int c = 256 * i + 4 * l;
    if (c < D) {
      const f4 g = *reinterpret_cast<const f4*>(p.gamma + c), be = *reinterpret_cast<const f4*>(p.beta + c);
      store4(static_cast<T*>(p.Y) + row * D + c, (x[i] - splat(mean)) * rstd * g + be);
    }
  }
  if (l == 0) {
    p.stats[2 * row] = mean;
    p.stats[2 * row + 1] = rstd;
  }
}

template <typename T, int F, int NCH>
__global__ __launch_bounds__(256) void post_norm_bwd_kernel(PostNormParams p) {
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const long long rows = (long long)p.B * p.L;
  const int D = p.H * F;
  __shared__ float red[4][2][256 * NCH];
  f4 aw[NCH], ab[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    aw[i] = splat(0.f);
    ab[i] = splat(0.f);
  }
  const long long r0 = (long long)blockIdx.x * kRowsPerBlockBwd;
  for (long long row = r0 + wave; row < r0 + kRowsPerBlockBwd && row < rows; row += 4) {
    const int b = (int)(row / p.L), t = (int)(row - (long long)b * p.L);
    const float mean = p.stats[2 * row], rstd = p.stats[2 * row + 1];
    f4 xh[NCH], g[NCH];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = 256 * i + 4 * l;
      const bool act = c < D;
      const int h = c / F, f = c - h * F;
      const f4 x = ld4(static_cast<const T*>(p.X) + (((size_t)b * p.H + h) * p.L + t) * F + f, act);
      const f4 dy = ld4(static_cast<const T*>(p.dY) + row * D + c, act);
      const f4 ga = act ? *reinterpret_cast<const f4*>(p.gamma + c) : splat(0.f);
      xh[i] = (x - splat(mean)) * rstd;
      g[i] = dy * ga;
      aw[i] += dy * xh[i];
      ab[i] += dy;
      s1 += hsum(g[i]);
      s2 += hsum(g[i] * xh[i]);
    }
    const float m1 = sum_wave(s1) / (float)D, m2 = sum_wave(s2) / (float)D;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = 256 * i + 4 * l;
      if (c < D) {
        const int h = c / F, f = c - h * F;
        store4(static_cast<T*>(p.dX) + (((size_t)b * p.H + h) * p.L + t) * F + f,
               (g[i] - splat(m1) - xh[i] * m2) * rstd);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = 256 * i + 4 * l;
    if (c < D) {
      *reinterpret_cast<f4*>(&red[wave][0][c]) = aw[i];
      *reinterpret_cast<f4*>(&red[wave][1][c]) = ab[i];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < 2 * D; c += 256) {
    const int k = c / D, j = c - k * D;
    p.partial[((size_t)blockIdx.x * 2 + k) * D + j] = ((red[0][k][j] + red[1][k][j]) + red[2][k][j]) + red[3][k][j];
  }
}

int layer_io_bwd_blocks(int B, int L) {
  const long long rows = (long long)B * L;
  return (int)((rows + kRowsPerBlockBwd - 1) / kRowsPerBlockBwd);
}
int layer_io_max_width() { return kMaxD; }

template <typename T, int F>
static hipError_t launch_producer_t(const ProducerParams& p, bool bwd, hipStream_t stream) {
  const long long rows = (long long)p.B * p.L;
  const dim3 grid(layer_io_bwd_blocks(p.B, p.L)), block(256);
  const int D = p.H * F;  // the backwards' per-lane arrays cover D in 256-feature chunks
  if (bwd && D <= 256)
    hipLaunchKernelGGL((qkvu_producer_bwd_kernel<T, F, 1>), grid, block, 0, stream, p);
  else if (bwd && D <= 512)
    hipLaunchKernelGGL((qkvu_producer_bwd_kernel<T, F, 2>), grid, block, 0, stream, p);
  else if (bwd)
    hipLaunchKernelGGL((qkvu_producer_bwd_kernel<T, F, kMaxD / 256>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((qkvu_producer_fwd_kernel<T, F>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_producer(const ProducerParams& p, int dtype, bool bwd, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_producer_t<__bf16, 64>(p, bwd, stream);
    if (p.F == 32) return launch_producer_t<__bf16, 32>(p, bwd, stream);
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_producer_t<_Float16, 64>(p, bwd, stream);
    if (p.F == 32) return launch_producer_t<_Float16, 32>(p, bwd, stream);
  } else {
    if (p.F == 64) return launch_producer_t<float, 64>(p, bwd, stream);
    if (p.F == 32) return launch_producer_t<float, 32>(p, bwd, stream);
  }
  return hipErrorInvalidValue;
}

template <typename T, int F>
static hipError_t launch_post_norm_t(const PostNormParams& p, bool bwd, hipStream_t stream) {
  const long long rows = (long long)p.B * p.L;
  const dim3 grid(layer_io_bwd_blocks(p.B, p.L)), block(256);
  const int D = p.H * F;
  if (bwd && D <= 256)
    hipLaunchKernelGGL((post_norm_bwd_kernel<T, F, 1>), grid, block, 0, stream, p);
  else if (bwd && D <= 512)
    hipLaunchKernelGGL((post_norm_bwd_kernel<T, F, 2>), grid, block, 0, stream, p);
  else if (bwd)
    hipLaunchKernelGGL((post_norm_bwd_kernel<T, F, kMaxD / 256>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((post_norm_fwd_kernel<T, F>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_post_norm(const PostNormParams& p, int dtype, bool bwd, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_post_norm_t<__bf16, 64>(p, bwd, stream);
    if (p.F == 32) return launch_post_norm_t<__bf16, 32>(p, bwd, stream);
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_post_norm_t<_Float16, 64>(p, bwd, stream);
    if (p.F == 32) return launch_post_norm_t<_Float16, 32>(p, bwd, stream);
  } else {
    if (p.F == 64) return launch_post_norm_t<float, 64>(p, bwd, stream);
    if (p.F == 32) return launch_post_norm_t<float, 32>(p, bwd, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
