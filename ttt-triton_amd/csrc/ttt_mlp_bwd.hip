// TTT-MLP backward on gfx950: a reverse sweep per chain and a dXQ/dXK pass.
//
// 1. mlp_bwd_kernel: one workgroup of NW wavefronts per (batch, head) chain,
//    wave w owning HT hidden tiles S = [16 HT w, 16 HT (w+1)) (HT = 4, or
//    four waves of one tile for FF = F = 64, as in the forward), walks the sequence
//    in reverse and carries the gradient wrt the state, dW1, db1, dW2, db2.
//    Inputs besides the sequence: the forward's final W2 and its saved
//    buffer, which holds for every mini-batch the state-update
//    operands and the activations the gradient needs (MlpSavedSlot): nothing
//    of the forward is recomputed (ops/ttt_mlp.py:9-67 differentiated by hand).
//    The products with W1 (dXQ += dZ1b W1^T, dXK += dZ1 W1^T) do not feed the
//    recurrence, so this pass hands dZ1b and dZ1 over instead (MlpBwdWsSlot)
//    and never needs W1.
// 2. the dXQ/dXK pass: one wave per (chain, checkpoint group, feature tile),
//    all independent: it walks its group forward from the checkpoint, W1^T in
//    registers, and forms dXQ and dXK.  With one wave per feature tile per
//    chain (NW == F/16) and a CU to spare per chain, it runs inside the
//    sweep's launch on the CUs the 192-odd sweeps leave idle, group by group
//    as the sweeps publish them (mlp_bwd_dx_worker); otherwise it is a second
//    launch (mlp_bwd_dx_kernel).
//
// In the reverse sweep W2 is needed (the gradient flows through products with
// it): W2^T [F][FF] lives in LDS in fp32, columns XOR-swizzled so both access
// shapes are bank-conflict free, rebuilt per mini-batch as W2_s = W2_{s+1} +
// X2_s^T (e G2_s) from the exact operands the forward's update used, starting
// from the final state: the rebuild undoes each update up to fp32 rounding, so
// no checkpoint reload is needed (kernels/mlp_backward.py:340 instead restarts
// every checkpoint group; the algorithm and data flow here are our own).  dW1 is accumulated in LDS as dW1^T [FF][F], so both
// orientations it is read in are direct LDS reads; dW2 lives in the MFMA
// accumulator registers.  Each wave only touches its own hidden rows/columns
// of these, so no barrier guards them.
//
// Row-wise work on [16 x F] tiles (LayerNorm backwards) is done redundantly by
// every wave.  Contractions over the hidden units are split by slice; their
// [16 x F] partials meet in one LDS exchange area, fenced by a barrier after
// the writes and one after the reads: four barriers per mini-batch.  The
// per-slice [16 x 64] temporaries are consumed in the order they are made (dX2
// folds into dZ1, dG1 into dP and dZ1, the -e Q2 share straight into the
// exchange area) so that the loop runs without spilling.
#include <type_traits>

#include "ttt_buf.h"
#include "ttt_eta.h"
#include "ttt_kernels.h"
#include "ttt_ln.h"

namespace ttt {

// Exchange area, in lane order (f4 per lane), byte offsets:
//   [16 x F] partials of wave w, feature tile c   at (w * FT + c) * 1024
//   [16 x 16] partial k of wave w                 at PART + (k * NW + w) * 1024
//   after the second barrier the [16 x F] blocks hold the dXK partials
template <int FT, int NW> struct MlpBwdExchange {
  static constexpr int PART = NW * FT * 1024;
  static constexpr int BYTES = (NW * FT + 3 * NW) * 1024;
  f4 mem[BYTES / 16];
};

// The inner-loss LayerNorm backward is split over the waves by token rows
// when there are four waves and F = 64, as in the forward: wave w takes rows
// 4w..4w+3 with lane l on feature l, and the rows of dZ2 and dtgt meet in the
// exchange area's [16 x 16] partial region, which is free from the barrier
// after the dN1 / de / dG2 partials are read until the next mini-batch (dZ2 in
// C layout and as the transposed operand frags of its products, dtgt in C
// layout for the tile owners).
template <int FT, int NW> constexpr bool kBwdRowSplit = (NW == 4 && FT == 4);
// In bf16 the readout LayerNorm's backward (dZ2b from dout) is split the same
// way; its rows meet in a region of their own (dZ2b in bf16 C-layout tiles,
// then per-wave column sums), written after the last barrier of a mini-batch
// and read after the first of the next, so no other phase touches it.
constexpr int kRsL = 3072, kRsLCol = 2048;

template <int FT, int NW, int HT> struct MlpBwdShared {
  float w2t[16 * FT * 16 * HT * NW];   // W2^T [F][FF], 16 x 16 blocks (LdsMat)
  float dw1t[16 * FT * 16 * HT * NW];  // dW1^T [FF][F], 16 x 16 blocks (LdsMat)
  MlpBwdExchange<FT, NW> x;
  float lnw[16 * FT], lnb[16 * FT];  // LayerNorm parameters of the chain's head
  alignas(16) unsigned char lx[kBwdRowSplit<FT, NW> ? kRsL : 16];  // readout LayerNorm rows (row split, bf16)
};

constexpr int kRsDz2 = 0, kRsDtgt = 4096, kRsDz2T = 8192;  // byte offsets in the partial region

typedef __attribute__((address_space(3))) unsigned short lds_u16;
typedef __attribute__((address_space(3))) bf4 lds_bf4;
// element (row 4w + j, feature 16 lo + n) of a [16 x F] matrix into its
// transposed operand frags (free = row, k = feature): element n & 3 of frag
// lane 16 (n >> 2) + 4w + j of tile lo.  16-bit frags sit in the skewed 8-byte
// slots of lds::tfrag16_slot (csrc/ttt_lds_layout.h), so that neither the
// element writes nor the frag reads conflict; fp32 frags in tiles of 64 lanes
// x 16 bytes in lane order.  tfrag_put_addr is the lane's address for j = 0.
template <typename T> __device__ __forceinline__ unsigned tfrag_put_addr(unsigned base, int lo, int w, int n) {
  if constexpr (sizeof(T) == 2)
    return base + 8u * (unsigned)lds::tfrag16_put_slot(lo, w, n) + 2u * (unsigned)(n & 3);
  else
    return base + 16u * (unsigned)(lo * 64 + 16 * (n >> 2) + 4 * w) + 4u * (unsigned)(n & 3);
}
template <typename T> __device__ __forceinline__ void lds_put_tfrag(unsigned a, int j, float v) {
  if constexpr (sizeof(T) == 2)
    *(lds_u16*)(uintptr_t)(a + 8u * j) = __builtin_bit_cast(unsigned short, (T)v);
  else
    *(lds_f32*)(uintptr_t)(a + 16u * j) = v;
}
template <typename T> __device__ __forceinline__ Frag<T> lds_get_tfrag(unsigned base, int c) {
  if constexpr (sizeof(T) == 2)
    return Frag<T>{__builtin_bit_cast(typename FragT<T>::type,
                                      *(lds_bf4*)(uintptr_t)(base + 8u * (unsigned)lds::tfrag16_slot(c, lane_id())))};
  else
    return Frag<T>{*(lds_f4*)(uintptr_t)(base + 16u * (unsigned)(c * 64 + lane_id()))};
}

size_t mlp_bwd_ws_slot_bytes(int F, int FF, int dtype) {
  const size_t t = dtype == TTT_DTYPE_F32 ? 4 : 2;
  return (size_t)2 * FF * 16 * t + (size_t)2 * F * 64;
}

// Control words of the fused dXQ/dXK workers: [0] next task, [1] set when a
// worker gave up waiting for a group, then one flag per (chain, checkpoint group).
constexpr int kDxCtrlHead = 4;
size_t mlp_bwd_ctrl_bytes(int B, int H, int NC, int G) {
  const size_t words = kDxCtrlHead + (size_t)B * H * ((NC + G - 1) / G);
  return (words * 4 + 255) & ~(size_t)255;
}

template <typename T, int FT, int NW, int HT>
__device__ __forceinline__ void mlp_bwd_dx_body(const MlpBwdParams& p, int chain, int kk, bool poison);

// Fused mode: workgroups B*H.. of the sweep's launch.  Each takes (chain,
// checkpoint group) tasks in the order the sweep finishes them (last group
// first), waits until the chain's sweep has published the group, and forms
// that group's dXQ/dXK (mlp_bwd_dx_body, wave = feature tile).  Blocks are
// dispatched in index order, so a worker only becomes resident after every
// sweep workgroup has; the sweeps never wait for the workers, so every wait
// ends.  Should that ordering not hold, a wait that exceeds p.dx_max_polls
// polls (s_sleep 8 between polls; the default, 2^22, is about a second
// against ~2 ms for a whole sweep) gives up: the worker raises the timeout
// word and writes NaN into that group's dXQ and dXK rows instead of reading a
// handoff that was never published, so the failure is visible in the output
// and through ttt_mlp_bwd_check, never silent.
//
// Visibility across XCDs without cache maintenance: the sweep writes the
// handoff with device-coherent (sc1, written-through) stores, waits for them
// to be acknowledged, then raises the group's flag with a device-scope
// store; the worker polls the flag with device-scope loads and reads the
// handoff with device-coherent (sc1) loads, which no stale L1 or L2 line
// serves.  Neither side writes back or invalidates a whole L2.
template <typename T, int FT, int NW, int HT>
__device__ __forceinline__ void mlp_bwd_dx_worker(const MlpBwdParams& p) {
  __shared__ int task_sh, gave_up_sh;
  const int nchain = p.B * p.H, ntask = nchain * p.NK;
  int* __restrict__ flags = p.dx_ctrl + kDxCtrlHead;
  for (;;) {
    if (threadIdx.x == 0) task_sh = atomicAdd(p.dx_ctrl, 1);
    __syncthreads();
    const int t = task_sh;
    __syncthreads();  // every wave has read the task before thread 0 takes the next
    if (t >= ntask) return;
    const int kk = p.NK - 1 - t / nchain, chain = t - (t / nchain) * nchain;
    if (threadIdx.x == 0) {
      int polls = 0, gave_up = 0;
      while (__hip_atomic_load(flags + chain * p.NK + kk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
        if (++polls > p.dx_max_polls) {
          __hip_atomic_store(p.dx_ctrl + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          gave_up = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(8);
      }
      gave_up_sh = gave_up;
    }
    __syncthreads();  // the group's flag was seen (its handoff stores are complete), or the wait gave up
    const bool poison = gave_up_sh != 0;
    mlp_bwd_dx_body<T, FT, NW, HT>(p, chain, kk, poison);
  }
}

template <typename T, int FT, int NW, int HT, bool LR, typename ET = T>
__global__ __launch_bounds__(64 * NW) void mlp_bwd_kernel(MlpBwdParams p) {
  if constexpr (NW == FT) {
    if ((int)blockIdx.x >= p.B * p.H) {
      mlp_bwd_dx_worker<T, FT, NW, HT>(p);
      return;
    }
  }
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  constexpr int FF = 16 * HT * NW;  // HT hidden tiles per wave
  constexpr float invF = 1.0f / F;
  constexpr int ST = (int)sizeof(T);
  constexpr int SE = (int)sizeof(ET);  // dense eta element
  using Slot = MlpSavedSlot<F, FF, ST>;
  __shared__ MlpBwdShared<FT, NW, HT> sh;

  const int chain = blockIdx.x;
  const int h = chain % p.H;
  const int NC = p.NC, G = p.G, NK = p.NK;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform
  const int l = lane_id(), g = l >> 4, n = l & 15;
  const int hs = 16 * HT * wave;

  // per-chain slabs as buffer resources; lane offsets shared by all of them
  const size_t xoff = (size_t)chain * NC * K * F;
  const size_t eoff = (size_t)chain * NC * K * K;
  const unsigned xbytes = (unsigned)((size_t)NC * K * F * ST), ebytes = (unsigned)((size_t)NC * K * K * SE);
  const rsrc_t rXQ = make_rsrc(static_cast<const T*>(p.XQ) + xoff, xbytes);
  const rsrc_t rXK = make_rsrc(static_cast<const T*>(p.XK) + xoff, xbytes);
  const rsrc_t rXV = make_rsrc(static_cast<const T*>(p.XV) + xoff, xbytes);
  const rsrc_t rDO = make_rsrc(static_cast<const T*>(p.dout) + xoff, xbytes);
  // eta and its gradient: dense [NC][K][K] blocks, or (LR) lr and dlr [NC][K] fp32
  const unsigned lbytes = (unsigned)(NC * K * 4);
  const rsrc_t rET = LR ? make_rsrc(static_cast<const float*>(p.eta) + (size_t)chain * NC * K, lbytes)
                        : make_rsrc(static_cast<const ET*>(p.eta) + eoff, ebytes);
  const rsrc_t rDXV = make_rsrc(static_cast<T*>(p.dXV) + xoff, xbytes);
  const rsrc_t rDET = LR ? make_rsrc(static_cast<float*>(p.deta) + (size_t)chain * NC * K, lbytes)
                         : make_rsrc(static_cast<ET*>(p.deta) + eoff, ebytes);
  const int eta_rule = p.eta_rule;
  const int xl = (n * F + 4 * g) * ST;        // frag lane offset in a [16 x F] block
  const int el = (n * K + 4 * g) * SE;        // frag lane offset in a [16 x 16] eta block
  const int en = (4 * g * K + n) * SE;        // eta[4g + j][n]: + j * K * SE
  const int e4 = ((K - 1) * K + 4 * g) * SE;  // eta[K-1][4g .. 4g+3]
  auto xs = [&](int s) { return s * K * F * ST; };
  auto es = [&](int s) { return s * K * K * SE; };

  // the forward's saved values of this chain, [NC] slots
  const rsrc_t rSV = make_rsrc(static_cast<const char*>(p.saved) + (size_t)chain * NC * Slot::BYTES,
                               (unsigned)(NC * Slot::BYTES));
  const int hl = ((wave * HT) * 64 + l) * 4 * ST;  // + o * 256 * ST: this wave's [16 x 64] slice, lane order
  const int fl = l * 4 * ST;                       // + c * 256 * ST: [16 x F] frags, lane order
  const int f4l = l * 16;                          // + c * 1024: fp32 tiles, lane order
  const int a2l = (4 * g * 16 + n) * 4;            // C-layout tile of a row-major [16 x 16] fp32 block
  const int a2tl = (n * 16 + 4 * g) * 4;           // the same block transposed (row n, columns 4g..4g+3)

  // handoff to the dXQ/dXK pass, [NC] slots of this chain
  using WS = MlpBwdWsSlot<F, FF, ST>;
  const rsrc_t rWS = make_rsrc(static_cast<char*>(p.ws) + (size_t)chain * NC * WS::BYTES, (unsigned)(NC * WS::BYTES));

  // W2 checkpoints [NK][...] and the final W2 of this chain
  const rsrc_t rW2l = make_rsrc(p.W2_last + (size_t)chain * FF * F, (unsigned)(FF * F * 4));
  const int w1l = ((4 * g) * FF + hs + n) * 4;  // [F][FF] tile lane offset, columns hs + ...
  const int w2l = ((hs + 4 * g) * F + n) * 4;   // [FF][F] tile lane offset, rows hs + ...

  // exchange-area lane slots: all blocks, this wave's [16 x F] blocks, this
  // wave's [16 x 16] blocks
  using Xch = MlpBwdExchange<FT, NW>;
  LdsLane xa(sh.x.mem, 0), xw(sh.x.mem, wave * FT * 1024), xs16(sh.x.mem, Xch::PART + wave * 1024);
  // row split: lane l on feature l of rows 4*wave + j; xr.get(b * 1024) reads
  // slot 16 wave + n of block b + l / 16, i.e. those rows of a lane-order tile set
  constexpr bool RS = kBwdRowSplit<FT, NW>;
  constexpr bool RSL = RS && ST == 2;
  const int lo = l >> 4;
  const int srow = (lo * 64 + 16 * wave + n) * 16;
  LdsLane xr(sh.x.mem, 768 * lo + 256 * wave);
  const unsigned dz2t_base = (unsigned)(uintptr_t)(lds_f32*)sh.x.mem + (unsigned)(Xch::PART + kRsDz2T);
  const unsigned dz2t_put = tfrag_put_addr<T>(dz2t_base, lo, wave, n);
  static_assert(!RS || kRsDz2T + (sizeof(T) == 2 ? lds::tfrag16_bytes(FT) : 16 * 64 * FT) <= 3 * NW * 1024,
                "transposed dZ2 frags within the partial region");

  // gradient wrt the state after the current mini-batch (this wave's slice):
  // dW2[S, :] in registers, dW1[:, S] in LDS (below)
  Tile dW2[HT][FT];
  float db1[HT], db2[FT];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < HT; ++o) dW2[o][i].v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int o = 0; o < HT; ++o) db1[o] = 0.f;
#pragma unroll
  for (int o = 0; o < FT; ++o) db2[o] = 0.f;
  // LDS views (this wave's hidden columns of W2^T, its hidden rows of dW1^T)
  // (W2 kept by rows instead, which swaps the two access shapes, measured
  // 9% slower at four hidden tiles per wave and no faster at one)
  LdsMat<FF> W2t(sh.w2t, hs);
  LdsMat<F> dW1s(sh.dw1t + hs * F, 0);
  // dW1 tile [F block q x hidden block o] (C layout), also its frag (free = hidden, k = feature)
  auto dw1_get = [&](int q, int o) {
    Tile t;
    t.v = dW1s.row4(16 * o, 16 * q);
    return t;
  };
  auto dw1_put = [&](int q, int o, Tile t) { dW1s.put_row4(16 * o, 16 * q, t.v); };
  // dW1^T frag (free = feature block q, k = hidden block o)
  auto dw1T_frag = [&](int q, int o) { return to_frag<T>(dW1s.tile(16 * o, 16 * q).v); };
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int o = 0; o < HT; ++o) dw1_put(i, o, Tile{f4{0.f, 0.f, 0.f, 0.f}});
  // W2 tile [hidden block o x F block c] (C layout): frag (free = feature, k = hidden)
  auto w2_tile = [&](int o, int c) {
    Tile t;
    t.v = W2t.row4(16 * c, 16 * o);
    return t;
  };
  auto w2_put = [&](int o, int c, Tile t) { W2t.put_row4(16 * c, 16 * o, t.v); };
  // W2^T frag (free = hidden block o, k = feature block c)
  auto w2T_frag = [&](int o, int c) { return to_frag<T>(W2t.tile(16 * c, 16 * o).v); };
  // keep the gradient accumulators in the MFMA accumulator registers
  auto pin_dW = [&]() {
#pragma unroll
    for (int q_ = 0; q_ < FT; ++q_)
#pragma unroll
      for (int o_ = 0; o_ < HT; ++o_) asm volatile("" : "+a"(dW2[o_][q_].v));
  };
  // saved activations
  auto ld_hid = [&](int o, int off, int us) { return frag_to_f4(bload_frag<T>(rSV, hl + o * 256 * ST, us + off)); };
  auto ld_f32 = [&](int c, int off, int us) { return bload_frag<float>(rSV, f4l + c * 1024, us + off).v; };

  // LayerNorm parameters of this head, staged in LDS once and re-read where used
  for (int i = threadIdx.x; i < F; i += 64 * NW) {
    sh.lnw[i] = p.ln_w[(size_t)h * F + i];
    sh.lnb[i] = p.ln_b[(size_t)h * F + i];
  }
  auto ln_param = [&](const float* src, float (&v)[FT]) {
#pragma unroll
    for (int o = 0; o < FT; ++o) v[o] = src[16 * o + n];
  };
  const Frag<T> I = identity_frag<T>();

  float dlnw[FT], dlnb[FT];  // LN-parameter gradient partials (wave 0)
#pragma unroll
  for (int o = 0; o < FT; ++o) {
    dlnw[o] = 0.f;
    dlnb[o] = 0.f;
  }
  // row split: the LayerNorm parameter gradient partials of feature l over
  // this wave's rows (the parameters themselves are re-read from LDS where used)
  float dlnw_l = 0.f, dlnb_l = 0.f;

  // inputs of the first phase of a mini-batch, requested one mini-batch ahead
  Frag<T> nxq[FT], nxk[FT], nx2f[HT], ng2e[FT];
  auto prefetch = [&](int s) {
    const int u = s * Slot::BYTES;
#pragma unroll
    for (int q = 0; q < FT; ++q) {
      nxq[q] = bload_frag<T>(rXQ, xl + 16 * q * ST, xs(s));
      nxk[q] = bload_frag<T>(rXK, xl + 16 * q * ST, xs(s));
      ng2e[q] = bload_frag<T>(rSV, fl + q * 256 * ST, u + Slot::G2E);
    }
#pragma unroll
    for (int o = 0; o < HT; ++o) nx2f[o] = bload_frag<T>(rSV, hl + o * 256 * ST, u + Slot::X2);
  };
  prefetch(NC - 1);
  // W2 (this slice) after the last mini-batch; each step below rebuilds the
  // state entering it exactly from the saved update operands, so the
  // checkpoints are not needed here (rounding drift over a whole sequence is
  // a few fp32 ulps of W2)
#pragma unroll
  for (int i = 0; i < HT; ++i)
#pragma unroll
    for (int o = 0; o < FT; ++o) w2_put(i, o, bload_tile(rW2l, w2l, 0, F, 16 * i, 16 * o));
  // retire the loads issued so far: pending on loop entry, they make the
  // wait-count pass wait for every outstanding access in each iteration
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // the LayerNorm parameters are in LDS

  // Reverse sweep.  Regions between barriers:   A..P | B2a | LN2..B2b | B3
  // exchange area:                              dG2, dN1, de partials; dXQ, dXK partials
  for (int s = NC - 1; s >= 0; --s) {
    {
      const int us = s * Slot::BYTES;
      const int ws_ = s * WS::BYTES;
      pin_dW();
      W2t.pin();
      dW1s.pin();
      xa.pin();
      xw.pin();
      xs16.pin();

      // inputs of the readout LayerNorm backward, requested before the state
      // rebuild so that it hides their latency
      // (eta raw: converted where first used, so that the conversion does not
      // wait for the load here)
      // dense: eta[n][4g+j] ([t_k x t_q]) and eta[4g+j][n] ([t_q x t_k]);
      // LR: lr[4g .. 4g+3] and lr[n]
      Frag<ET> etaT_r, etan_r;
      f4 lr4;
      float lrn;
      if constexpr (LR) {
        lr4 = bload_frag<float>(rET, 16 * g, s * K * 4).v;
        lrn = bload_f32(rET, 4 * n, s * K * 4);
      } else {
        etaT_r = bload_frag<ET>(rET, el, es(s));
        etan_r = bload_ctile<ET>(rET, en, es(s), K);
      }
      // dout of this wave's feature tile for B3 (one tile per wave when NW >= FT)
      const Frag<T> dob = bload_frag<T>(rDO, xl + 16 * (wave % FT) * ST, xs(s));
      const f4 a2T = bload_tile(rSV, a2l, us + Slot::A2T, 16, 0, 0).v;  // A2^T [t_k x t_q]
      const f4 a2 = bload_frag<float>(rSV, a2tl, us + Slot::A2T).v;    // A2   [t_q x t_k]
      // (split by rows: dout, the normalised rows and their statistics of rows
      // 4*wave + j)
      const f4 rsb = bload_frag<float>(rSV, RSL ? (16 * wave + n) * 16 : f4l, us + Slot::RSB).v;
      f4 xhb[RSL ? 1 : FT], g2v[FT];
      Frag<T> dof[RSL ? 1 : FT];
      float lnw_tm[FT];
      ln_param(sh.lnw, lnw_tm);
      if constexpr (RSL) {
        xhb[0] = bload_frag<float>(rSV, srow, us + Slot::XHB).v;
        dof[0] = bload_ctile<T>(rDO, l * ST, xs(s) + 4 * wave * F * ST, F);
      }
#pragma unroll
      for (int c = 0; c < FT; ++c) {
        if constexpr (!RSL) {
          xhb[c] = ld_f32(c, Slot::XHB, us);
          dof[c] = bload_frag<T>(rDO, xl + 16 * c * ST, xs(s));
        }
        g2v[c] = ld_f32(c, Slot::G2, us);
      }

      Frag<T> xk[FT], xkTf[FT];
      f4 at = f4{0.f, 0.f, 0.f, 0.f}, a = f4{0.f, 0.f, 0.f, 0.f};
      Frag<T> x2f[HT];
      {
        Frag<T> xq[FT], g2e[FT];
#pragma unroll
        for (int q = 0; q < FT; ++q) {
          xq[q] = nxq[q];
          xk[q] = nxk[q];
          g2e[q] = ng2e[q];
        }
#pragma unroll
        for (int o = 0; o < HT; ++o) x2f[o] = nx2f[o];
#pragma unroll
        for (int q = 0; q < FT; ++q) xkTf[q] = to_frag<T>(transpose16(xk[q], I).v);
#pragma unroll
        for (int q = 0; q < FT; q += 2) {
          mma32(at, xk[q], xk[q + 1], xq[q], xq[q + 1]);  // A1^T [t_k x t_q]
          mma32(a, xq[q], xq[q + 1], xk[q], xk[q + 1]);   // A1   [t_q x t_k]
        }
        // ---- A: rebuild W2_s (this slice) from the forward's update operands;
        //      the tiles of one feature block are read before any is written
        //      back, so the LDS reads overlap
        //      (two register sets across feature blocks, as in the dW1 update,
        //      measured 2% slower here)
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          const Frag<T> ng = negate(g2e[c]);
          Tile w[HT];
#pragma unroll
          for (int o = 0; o < HT; ++o) w[o] = w2_tile(o, c);
#pragma unroll
          for (int o = 0; o < HT; ++o) mma16(w[o].v, x2f[o], ng);
#pragma unroll
          for (int o = 0; o < HT; ++o) w2_put(o, c, w[o]);
        }
      }

      // inputs of B1 and X, requested before the LayerNorm backward
      Frag<T> x2bs[HT], sp1bs[HT], g2es[FT];
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        x2bs[o] = bload_frag<T>(rSV, hl + o * 256 * ST, us + Slot::X2B);
        sp1bs[o] = bload_frag<T>(rSV, hl + o * 256 * ST, us + Slot::SP1B);
      }
#pragma unroll
      for (int c = 0; c < FT; ++c) g2es[c] = bload_frag<T>(rSV, fl + c * 256 * ST, us + Slot::G2E);

      // ---- L: readout layer 2 LayerNorm backward (every wave): dZ2b from dout
      Frag<T> dz2bf[FT], dz2bF[FT];
      float dz2b_cs[FT];  // column sums of dZ2b (fp32)
      if constexpr (RSL) {
        // rows 4*wave + j of feature l
        const f4 dT = frag_to_f4(dof[0]), xh = xhb[0];
        const f4 gy = dT * sh.lnw[l];
        const f4 s1 = sum4_wave(gy) * invF, s2 = sum4_wave(gy * xh) * invF;
        f4 dz;
        float aw = 0.f, ab = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          aw += dT[j] * xh[j];
          ab += dT[j];
          dz[j] = rsb[j] * (gy[j] - s1[j] - xh[j] * s2[j]);
        }
        dlnw_l += aw;
        dlnb_l += ab;
        const unsigned lxb = (unsigned)(uintptr_t)(lds_f32*)sh.lx;
        *(lds_bf4*)(uintptr_t)(lxb + 8u * (unsigned)lds::crow16_slot(lo, 16 * wave + n)) =
            __builtin_bit_cast(bf4, to_frag<T>(dz).v);
        *(lds_f32*)(uintptr_t)(lxb + kRsLCol + 4u * (unsigned)(wave * 64 + n * 4 + lo)) = dz[0] + dz[1] + dz[2] + dz[3];
        __syncthreads();  // (L) the rows of dZ2b of every wave in
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          dz2bf[c].v = __builtin_bit_cast(typename FragT<T>::type,
                                          *(lds_bf4*)(uintptr_t)(lxb + 8u * (unsigned)lds::crow16_slot(c, l)));
          dz2bF[c] = to_frag<T>(transpose16(dz2bf[c], I).v);
        }
        f4 cs = f4{0.f, 0.f, 0.f, 0.f};  // column sums of features 16c + n
#pragma unroll
        for (int w = 0; w < NW; ++w) cs += *(lds_f4*)(uintptr_t)(lxb + kRsLCol + 16u * (unsigned)(w * 16 + n));
#pragma unroll
        for (int c = 0; c < FT; ++c) dz2b_cs[c] = cs[c];
      } else {
        f4 gy[FT];
        f4 s1 = f4{0.f, 0.f, 0.f, 0.f}, s2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          const f4 dT = transpose16(dof[c], I).v;  // dout, token-major
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            gy[c][j] = dT[j] * lnw_tm[c];
            s1[j] += gy[c][j];
            s2[j] += gy[c][j] * xhb[c][j];
          }
          if (wave == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              dlnw[c] += dT[j] * xhb[c][j];
              dlnb[c] += dT[j];
            }
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s1[j] = sum_row16(s1[j]) * invF;
          s2[j] = sum_row16(s2[j]) * invF;
        }
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          f4 dz;
          float cs = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dz[j] = rsb[j] * (gy[c][j] - s1[j] - xhb[c][j] * s2[j]);
            cs += dz[j];
          }
          dz2b_cs[c] = sum_col4(cs);
          dz2bf[c] = to_frag<T>(dz);
          dz2bF[c] = to_frag<T>(transpose16(dz2bf[c], I).v);
        }
      }
      const f4 etaT = LR ? eta_rowfrag_from_lr(eta_rule, lr4) : frag_to_f4(etaT_r);
      const f4 eta_n = LR ? eta_ctile_from_lr(eta_rule, lrn) : frag_to_f4(etan_r);
      // dN2 = -dZ2b G2^T (both layouts): deta part, dA2
      f4 detT, dA2T, dA2;
      Frag<T> m2f;  // -(eta o A2 + eta) for wave 0, zero for the others
      {
        f4 m2;
#pragma unroll
        for (int j = 0; j < 4; ++j) m2[j] = eta_n[j] * a2[j] + eta_n[j];
        m2f = to_frag<T>(wave == 0 ? -m2 : f4{0.f, 0.f, 0.f, 0.f});
      }
      {
        Frag<T> g2F[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) g2F[c] = to_frag<T>(transpose16(to_frag<T>(g2v[c]), I).v);
        f4 dn = f4{0.f, 0.f, 0.f, 0.f}, dnT = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < FT; c += 2) {
          mma32(dn, dz2bF[c], dz2bF[c + 1], g2F[c], g2F[c + 1]);   // dZ2b G2^T [t_q x t_k]
          mma32(dnT, g2F[c], g2F[c + 1], dz2bF[c], dz2bF[c + 1]);  // G2 dZ2b^T [t_k x t_q]
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          detT[j] = -dnT[j] * (1.0f + a2T[j]);
          dA2T[j] = -dnT[j] * etaT[j];
          dA2[j] = -dn[j] * eta_n[j];
        }
      }
      pin_dW();

      // inputs of the layer-1 gradient phases (G1, gelu'(Z1), Pm gelu''(Z1)),
      // requested a phase ahead
      Frag<T> g1s[HT], sp1s[HT], h1s[HT];
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        g1s[o] = bload_frag<T>(rSV, hl + o * 256 * ST, us + Slot::G1);
        sp1s[o] = bload_frag<T>(rSV, hl + o * 256 * ST, us + Slot::SP1);
        h1s[o] = bload_frag<T>(rSV, hl + o * 256 * ST, us + Slot::H1);
      }
      // ---- B1: readout layer 1 backward (per slice): dZ1b, and dX2 = dA2^T X2b
      Frag<T> dz1bf[HT];
      float dz1b_cs[HT];  // column sums of dZ1b (fp32)
      Tile dX2[HT];
      {
        const Frag<T> dA2Tf = to_frag<T>(dA2T), dA2f = to_frag<T>(dA2);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          const Frag<T> x2bf = x2bs[o];
          const f4 sp1b = frag_to_f4(sp1bs[o]);
          f4 dx2b = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < FT; c += 2) mma32(dx2b, dz2bF[c], dz2bF[c + 1], w2T_frag(o, c), w2T_frag(o, c + 1));
          mma16(dx2b, dA2Tf, x2f[o]);  // + dA2 X2
          const f4 dz = dx2b * sp1b;
          dz1b_cs[o] = sum_col4(dz[0] + dz[1] + dz[2] + dz[3]);
          dz1bf[o] = to_frag<T>(dz);
          dX2[o].v = f4{0.f, 0.f, 0.f, 0.f};
          mma16(dX2[o].v, dA2f, x2bf);  // dA2^T X2b
        }
      }
      // ---- X: dX2 += (-e G2) dW2'^T (contraction over features; dW2'^T frags by
      //      transposes; dW2' is the gradient wrt the state after s, not yet updated)
      {
        Frag<T> eg2F[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c)
          eg2F[c] = to_frag<T>(transpose16(g2es[c], I).v);
#pragma unroll
        for (int o = 0; o < HT; ++o)
#pragma unroll
          for (int c = 0; c < FT; c += 2) {
            const Frag<T> u0 = to_frag<T>(transpose16(to_frag<T>(dW2[o][c].v), I).v);
            const Frag<T> u1 = to_frag<T>(transpose16(to_frag<T>(dW2[o][c + 1].v), I).v);
            mma32(dX2[o].v, eg2F[c], eg2F[c + 1], u0, u1);
          }
      }
      // ---- N: dN1 = dZ1b G1^T (both layouts), partial over this slice
      {
        Frag<T> g1F[HT];
#pragma unroll
        for (int o = 0; o < HT; ++o)
          g1F[o] = to_frag<T>(transpose16(g1s[o], I).v);
        Frag<T> dz1bF[HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          dz1bF[o] = to_frag<T>(transpose16(dz1bf[o], I).v);
          bstore_frag_dev<T>(rWS, hl + o * 256 * ST, ws_ + WS::DZ1BF, dz1bF[o]);
        }
        f4 dn = f4{0.f, 0.f, 0.f, 0.f}, dnT = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o + 1 < HT; o += 2) {
          mma32(dn, dz1bF[o], dz1bF[o + 1], g1F[o], g1F[o + 1]);
          mma32(dnT, g1F[o], g1F[o + 1], dz1bF[o], dz1bF[o + 1]);
        }
        if constexpr (HT & 1) {
          mma16(dn, dz1bF[HT - 1], g1F[HT - 1]);
          mma16(dnT, g1F[HT - 1], dz1bF[HT - 1]);
        }
        xs16.put(0, dn);
        xs16.put(NW * 1024, dnT);
      }
      f4 g2p[FT];  // G2, for P and the layer-2 state gradient
#pragma unroll
      for (int c = 0; c < FT; ++c) g2p[c] = ld_f32(c, Slot::G2, us);
      // ---- Q: dG1 = -M1^T dZ1b - e (XK dW1' + db1'), then at once
      //      dP = dG1 (.) gelu'(Z1) and dZ1 = dG1 (.) Pm gelu''(Z1) + dX2 (.) gelu'(Z1)
      //      (the dZ2 W2^T part of dX2 is added after the inner-loss backward)
      const f4 e = LR ? eta_lastrow_from_lr(bload_frag<float>(rET, 16 * g, s * K * 4).v)
                      : frag_to_f4(bload_frag<ET>(rET, e4, es(s)));
      Tile dZ1[HT];
      Frag<T> dPf[HT], dPF[HT];
      f4 dep = f4{0.f, 0.f, 0.f, 0.f};  // eta-row gradient partial (G1 . Q1 + G2 . Q2)
      {
        f4 m1;
#pragma unroll
        for (int j = 0; j < 4; ++j) m1[j] = eta_n[j] * a[j] + eta_n[j];
        const Frag<T> mf = to_frag<T>(-m1);
        // (the dW1' rows of hidden block o + 1 are read while block o's
        // products run)
        Tile dr[2][FT];
#pragma unroll
        for (int q = 0; q < FT; ++q) dr[0][q] = dw1_get(q, 0);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          if (o + 1 < HT) {
#pragma unroll
            for (int q = 0; q < FT; ++q) dr[(o + 1) & 1][q] = dw1_get(q, o + 1);
          }
          Tile(&cur)[FT] = dr[o & 1];
          f4 q1 = f4{db1[o], db1[o], db1[o], db1[o]};
#pragma unroll
          for (int q = 0; q < FT; q += 2) mma32(q1, xk[q], xk[q + 1], to_frag<T>(cur[q].v), to_frag<T>(cur[q + 1].v));
          f4 dg1 = f4{0.f, 0.f, 0.f, 0.f};
          mma16(dg1, mf, dz1bf[o]);
          const f4 g1 = frag_to_f4(g1s[o]), sp = frag_to_f4(sp1s[o]), h1 = frag_to_f4(h1s[o]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dg1[j] -= e[j] * q1[j];
            dep[j] += g1[j] * q1[j];
          }
          dZ1[o].v = dg1 * h1 + dX2[o].v * sp;
          dPf[o] = to_frag<T>(dg1 * sp);
          dPF[o] = to_frag<T>(transpose16(dPf[o], I).v);
          db1[o] += dz1b_cs[o];  // db1' has been used
        }
      }
      // ---- P: Q2 = X2 dW2' + db2' per feature tile; dG2 partial over this slice:
      //      dP W2 - e Q2 (- M2^T dZ2b, which every wave holds, added once by wave 0)
      {
        Frag<T> x2F[HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) x2F[o] = to_frag<T>(transpose16(x2f[o], I).v);
        // (the W2 rows of feature block c + 1 are read while block c's products run)
        Tile wr[2][HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) wr[0][o] = w2_tile(o, 0);
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          if (c + 1 < FT) {
#pragma unroll
            for (int o = 0; o < HT; ++o) wr[(c + 1) & 1][o] = w2_tile(o, c + 1);
          }
          Tile(&wc)[HT] = wr[c & 1];
          f4 q2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int o = 0; o + 1 < HT; o += 2)
            mma32(q2, x2F[o], x2F[o + 1], to_frag<T>(dW2[o][c].v), to_frag<T>(dW2[o + 1][c].v));
          if constexpr (HT & 1) mma16(q2, x2F[HT - 1], to_frag<T>(dW2[HT - 1][c].v));
          // Q2 enters dG2 as -e Q2 and the eta-row gradient as G2 . Q2, both
          // linear in Q2: this slice's share goes into the partials as it is
          // (wave 0's share carries db2')
          if (wave == 0) q2 += f4{db2[c], db2[c], db2[c], db2[c]};
          const f4 g2 = g2p[c];
          f4 z;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dep[j] += g2[j] * q2[j];
            z[j] = -e[j] * q2[j];
          }
          mma16(z, m2f, dz2bf[c]);
#pragma unroll
          for (int o = 0; o + 1 < HT; o += 2) mma32(z, dPF[o], dPF[o + 1], to_frag<T>(wc[o].v), to_frag<T>(wc[o + 1].v));
          if constexpr (HT & 1) mma16(z, dPF[HT - 1], to_frag<T>(wc[HT - 1].v));
          xw.put(c * 1024, z);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) dep[j] = sum_row16(dep[j]);
        xs16.put(2 * NW * 1024, dep);
#pragma unroll
        for (int c = 0; c < FT; ++c) db2[c] += dz2b_cs[c];  // db2' has been used
      }
      // two terms of the layer-2 state gradient, X2b^T dZ2b + dP^T G2 (dW2' has
      // been used)
      {
        Frag<T> x2bf[HT];
#pragma unroll
        for (int o = 0; o < HT; ++o) x2bf[o] = x2bs[o];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          const Frag<T> g2f = to_frag<T>(g2p[c]);
#pragma unroll
          for (int o = 0; o < HT; ++o) mma32(dW2[o][c].v, x2bf[o], dPf[o], dz2bf[c], g2f);
        }
      }
      // inputs of the inner-loss backward and of B2b, requested before the barrier
      // (split by rows: the statistics of rows 4*wave + j, XV and XK rows)
      const int rsl = RS ? (16 * wave + n) * 16 : f4l;
      const f4 rstd2 = bload_frag<float>(rSV, rsl, us + Slot::RSTD).v;
      const f4 cc2 = bload_frag<float>(rSV, rsl, us + Slot::CC).v;
      f4 xh2[RS ? 1 : FT], g22[RS ? 1 : FT];
      Frag<T> xvf[RS ? 2 : FT], g1ef[HT];
      if constexpr (RS) {
        xh2[0] = bload_frag<float>(rSV, srow, us + Slot::XH).v;
        g22[0] = bload_frag<float>(rSV, srow, us + Slot::G2).v;
        xvf[0] = bload_ctile<T>(rXV, l * ST, xs(s) + 4 * wave * F * ST, F);
        xvf[1] = bload_ctile<T>(rXK, l * ST, xs(s) + 4 * wave * F * ST, F);
      } else {
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          xh2[c] = ld_f32(c, Slot::XH, us);
          g22[c] = ld_f32(c, Slot::G2, us);
          xvf[c] = bload_frag<T>(rXV, xl + 16 * c * ST, xs(s));
        }
      }
#pragma unroll
      for (int o = 0; o < HT; ++o) g1ef[o] = bload_frag<T>(rSV, hl + o * 256 * ST, us + Slot::G1E);
      float lnw2[FT], lnb2[FT];
      ln_param(sh.lnw, lnw2);
      ln_param(sh.lnb, lnb2);
      __syncthreads();  // (1) dG2, dN1, eta-row partials in

      // ---- B2a: assemble dN1, de; deta (wave 0); dG2
      f4 dA1T, dA1;
      Tile dG2[RS ? 1 : FT];  // row split: rows 4*wave + j of feature l
      {
        f4 dn1 = f4{0.f, 0.f, 0.f, 0.f}, dn1T = f4{0.f, 0.f, 0.f, 0.f}, de = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          dn1 += xa.get(Xch::PART + w * 1024);
          dn1T += xa.get(Xch::PART + (NW + w) * 1024);
          de += xa.get(Xch::PART + (2 * NW + w) * 1024);
        }
        if constexpr (RS) {
          dG2[0].v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int w = 0; w < NW; ++w) dG2[0].v += xr.get(w * FT * 1024);
        } else {
#pragma unroll
          for (int c = 0; c < FT; ++c) {
            dG2[c].v = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < NW; ++w) dG2[c].v += xa.get((w * FT + c) * 1024);
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dn1[j] = -dn1[j];
          dn1T[j] = -dn1T[j];
          detT[j] += dn1T[j] * (1.0f + at[j]);
          dA1T[j] = dn1T[j] * etaT[j];
          dA1[j] = dn1[j] * eta_n[j];
        }
        if (n == K - 1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) detT[j] -= de[j];
        }
        if constexpr (LR) {
          // dlr of columns 4g..4g+3: lane n == 0 of each group stores
          const f4 dl = dlr_from_detaT(eta_rule, detT);
          bstore_frag<float>(rDET, keep_or_drop(16 * g, wave == 0 && n == 0), s * K * 4, Frag<float>{dl});
        } else {
          bstore_frag<ET>(rDET, keep_or_drop(el, wave == 0), es(s), to_frag<ET>(detT));
        }
      }
      __syncthreads();  // (1x) exchange area free
      pin_dW();
      Frag<T> xqf[FT];  // XQ again (L2-resident), for the layer-1 state gradient
#pragma unroll
      for (int q = 0; q < FT; ++q) xqf[q] = bload_frag<T>(rXQ, xl + 16 * q * ST, xs(s));
      // ---- LN2: backward of G2 = ln_fused_l2_bwd(Z2, XV - XK) (every wave, or
      //      split by rows)
      f4 dz2[RS ? 1 : FT], dtgt[RS ? 1 : FT];
      if constexpr (RS) {
        // ln_fused_l2_bwd's backward for rows 4*wave + j (the same terms as
        // LnL2Lite::backward, with the row sums over the 64 lanes)
        const f4 xh = xh2[0], G = g22[0];
        const f4 tgt = frag_to_f4(xvf[0]) - frag_to_f4(xvf[1]);
        const float lnw_l = sh.lnw[l], lnb_l = sh.lnb[l];
        const f4 u = dG2[0].v * rstd2;
        const f4 mu_u = sum4_wave(u) * invF, mu_ux = sum4_wave(u * xh) * invF, dsig = -sum4_wave(u * G);
        f4 dxh, dtg;
        float aw = 0.f, ab = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float go = lnw_l * xh[j] + lnb_l - tgt[j];
          const float gx = go * lnw_l;
          const float d_gx = u[j] - mu_u[j] - xh[j] * mu_ux[j];
          const float d_go = d_gx * lnw_l;
          aw += d_gx * go + d_go * xh[j];
          ab += d_go;
          dtg[j] = -d_go;
          dxh[j] = -cc2[j] * u[j] - mu_ux[j] * gx + d_go * lnw_l;
        }
        dlnw_l += aw;
        dlnb_l += ab;
        const f4 m1 = sum4_wave(dxh) * invF, m2 = sum4_wave(dxh * xh) * invF;
        f4 dz;
#pragma unroll
        for (int j = 0; j < 4; ++j) dz[j] = rstd2[j] * (dxh[j] - m1[j] - xh[j] * m2[j]) + dsig[j] * xh[j] * invF;
        xr.put(Xch::PART + kRsDz2, dz);
        xr.put(Xch::PART + kRsDtgt, dtg);
#pragma unroll
        for (int j = 0; j < 4; ++j) lds_put_tfrag<T>(dz2t_put, j, dz[j]);
        bstore_ctile<T>(rDXV, l * ST, xs(s) + 4 * wave * F * ST, F, to_frag<T>(dtg));  // dXV rows
      } else {
        float lw_i[FT], lb_i[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          lw_i[c] = 0.f;
          lb_i[c] = 0.f;
        }
        float lnw_tm[FT], lnb_tm[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          lnw_tm[c] = lnw2[c];
          lnb_tm[c] = lnb2[c];
        }
        LnL2Lite<FT> ln2;
        ln2.rstd = rstd2;
        ln2.c = cc2;
        Tile G2[FT];
        f4 tgt[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          ln2.xh[c] = xh2[c];
          G2[c].v = g22[c];
          tgt[c] = transpose16(xvf[c], I).v - frag_to_f4(xkTf[c]);
        }
        ln2.backward(dG2, G2, tgt, lnw_tm, lnb_tm, dz2, dtgt, lw_i, lb_i);
        if (wave == 0) {
#pragma unroll
          for (int c = 0; c < FT; ++c) {
            dlnw[c] += lw_i[c];
            dlnb[c] += lb_i[c];
          }
        }
      }
      if constexpr (RS) __syncthreads();  // (1y) the rows of dZ2 and dtgt of every wave in
      // The checkpoint group that the previous mini-batch closed: this wave's
      // handoff stores for it (device-coherent, written through) have long been
      // issued, so waiting for them here costs little; barrier (2) then has
      // every wave's, and thread 0 raises the group's flag for the workers.
      // (Waiting right after a group's last stores stalls on their write-through;
      // an agent-scope release fence would also write back the whole L2.)
      const bool publish = p.dx_ctrl != nullptr && (s + 1) % G == 0 && s + 1 < NC;
      if (publish) __builtin_amdgcn_s_waitcnt(0);
      // ---- B2b: dZ2 into the state gradient and dX2; dZ1; dXQ and dXK partials
      Frag<T> dz1f[HT];
      {
        Frag<T> dz2F[FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          Frag<T> dz2f;
          if constexpr (RS) {
            const f4 z = xa.get(Xch::PART + kRsDz2 + c * 1024);
            dz2f = to_frag<T>(z);
            dz2F[c] = lds_get_tfrag<T>(dz2t_base, c);
            db2[c] += sum_col4(z[0] + z[1] + z[2] + z[3]);  // db2' was used in P
          } else {
            dz2f = to_frag<T>(dz2[c]);
            dz2F[c] = to_frag<T>(transpose16(dz2f, I).v);
          }
#pragma unroll
          for (int o = 0; o < HT; ++o) mma16(dW2[o][c].v, x2f[o], dz2f);  // + X2^T dZ2
        }
        Frag<T> dz1F[HT], eg1F[HT];
        // (the W2^T tiles of hidden block o + 1 are read while block o's
        // products run)
        Tile wt[2][FT];
#pragma unroll
        for (int c = 0; c < FT; ++c) wt[0][c] = W2t.tile(16 * c, 0);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          if (o + 1 < HT) {
#pragma unroll
            for (int c = 0; c < FT; ++c) wt[(o + 1) & 1][c] = W2t.tile(16 * c, 16 * (o + 1));
          }
          Tile(&cur)[FT] = wt[o & 1];
          f4 dx2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < FT; c += 2)
            mma32(dx2, dz2F[c], dz2F[c + 1], to_frag<T>(cur[c].v), to_frag<T>(cur[c + 1].v));
          dZ1[o].v += dx2 * frag_to_f4(sp1s[o]);
          dz1f[o] = to_frag<T>(dZ1[o].v);
          dz1F[o] = to_frag<T>(transpose16(dz1f[o], I).v);
          bstore_frag_dev<T>(rWS, hl + o * 256 * ST, ws_ + WS::DZ1F, dz1F[o]);
          eg1F[o] = to_frag<T>(transpose16(g1ef[o], I).v);
        }
        // dXK partial over this slice: (-e G1) dW1'^T (dW1' not yet updated);
        // the dW1'^T tiles of feature block f + 1 are read while block f's
        // products run
        {
          Tile tl[2][HT];
#pragma unroll
          for (int c = 0; c < HT; ++c) tl[0][c] = dW1s.tile(16 * c, 0);
#pragma unroll
          for (int f = 0; f < FT; ++f) {
            if (f + 1 < FT) {
#pragma unroll
              for (int c = 0; c < HT; ++c) tl[(f + 1) & 1][c] = dW1s.tile(16 * c, 16 * (f + 1));
            }
            Tile(&cur)[HT] = tl[f & 1];
            f4 zk_ = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c + 1 < HT; c += 2)
              mma32(zk_, eg1F[c], eg1F[c + 1], to_frag<T>(cur[c].v), to_frag<T>(cur[c + 1].v));
            if constexpr (HT & 1) mma16(zk_, eg1F[HT - 1], to_frag<T>(cur[HT - 1].v));
            xw.put(f * 1024, zk_);
          }
        }
      }
      Frag<T> xqTf[FT];
#pragma unroll
      for (int q = 0; q < FT; ++q) xqTf[q] = to_frag<T>(transpose16(xqf[q], I).v);
      prefetch(s > 0 ? s - 1 : 0);
      // the layer-1 state gradient: dW1 += XQ^T dZ1b + XK^T dZ1; biases
      // (two register sets, so that the reads of hidden block o + 1 are in
      // flight while block o's products and writes run)
      {
        Tile w[2][FT];
#pragma unroll
        for (int q = 0; q < FT; ++q) w[0][q] = dw1_get(q, 0);
#pragma unroll
        for (int o = 0; o < HT; ++o) {
          Tile(&cur)[FT] = w[o & 1];
          if (o + 1 < HT) {
#pragma unroll
            for (int q = 0; q < FT; ++q) w[(o + 1) & 1][q] = dw1_get(q, o + 1);
          }
#pragma unroll
          for (int q = 0; q < FT; ++q) mma32(cur[q].v, xqTf[q], xkTf[q], dz1bf[o], dz1f[o]);
#pragma unroll
          for (int q = 0; q < FT; ++q) dw1_put(q, o, cur[q]);
        }
      }
#pragma unroll
      for (int o = 0; o < HT; ++o) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += dZ1[o].v[j];
        db1[o] += sum_col4(acc);
      }
      if constexpr (!RS) {
#pragma unroll
        for (int c = 0; c < FT; ++c) {
          float acc = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc += dz2[c][j];
          db2[c] += sum_col4(acc);
        }
      }
      __syncthreads();  // (2) dXK partials in
      if (publish && threadIdx.x == 0)
        __hip_atomic_store(p.dx_ctrl + kDxCtrlHead + chain * NK + (s + 1) / G, 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);

      // ---- B3: the dXQ / dXK terms without W1 (to the handoff), dXV (tile owners)
      {
        const Frag<T> dA1Tf = to_frag<T>(dA1T), dA1f = to_frag<T>(dA1);
#pragma unroll
        for (int f = 0; f < FT; ++f) {
          if (f % NW != wave) continue;
          f4 dxq = transpose16(NW >= FT ? dob : dof[f], I).v;  // (f == wave when NW >= FT)
          const f4 dt = RS ? xa.get(Xch::PART + kRsDtgt + f * 1024) : dtgt[f];
          f4 dxk = -dt;
#pragma unroll
          for (int w = 0; w < NW; ++w) dxk += xa.get((w * FT + f) * 1024);
          mma16(dxq, dA1Tf, xkTf[f]);  // + dA1 XK
          mma16(dxk, dA1f, xqTf[f]);   // + dA1^T XQ
          bstore_frag_dev<float>(rWS, f4l + f * 1024, ws_ + WS::XQP, Frag<float>{dxq});
          bstore_frag_dev<float>(rWS, f4l + f * 1024, ws_ + WS::XKP, Frag<float>{dxk});
          if constexpr (!RS)
            bstore_frag<T>(rDXV, xl + 16 * f * ST, xs(s), to_frag<T>(transpose16(to_frag<T>(dt), I).v));
        }
      }
      __syncthreads();  // (2x) exchange area free for the next mini-batch
    }
  }
  if (p.dx_ctrl != nullptr) {
    // group 0, closed by the last mini-batch: every wave's handoff stores
    // acknowledged, then its flag
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_store(p.dx_ctrl + kDxCtrlHead + chain * NK, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- outputs: gradient wrt the initial state, LN parameters
  {
    const rsrc_t rdW1 = make_rsrc(p.dW1 + (size_t)chain * F * FF, (unsigned)(F * FF * 4));
    const rsrc_t rdW2 = make_rsrc(p.dW2 + (size_t)chain * FF * F, (unsigned)(FF * F * 4));
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int o = 0; o < HT; ++o) bstore_tile(rdW1, w1l, 0, FF, 16 * i, 16 * o, dw1_get(i, o));
#pragma unroll
    for (int i = 0; i < HT; ++i)
#pragma unroll
      for (int o = 0; o < FT; ++o) bstore_tile(rdW2, w2l, 0, F, 16 * i, 16 * o, dW2[i][o]);
    if (g == 0) {
#pragma unroll
      for (int o = 0; o < HT; ++o) p.db1[(size_t)chain * FF + hs + 16 * o + n] = db1[o];
    }
  }
  // row split: every wave's partials of feature l through the exchange area
  // (free since the last barrier of the sweep)
  float* const red = reinterpret_cast<float*>(sh.x.mem);
  if constexpr (RS) {
    red[wave * 64 + l] = dlnw_l;
    red[(NW + wave) * 64 + l] = dlnb_l;
    __syncthreads();
  }
  if (wave == 0) {
#pragma unroll
    for (int o = 0; o < FT; ++o) {
      float w = sum_col4(dlnw[o]);
      float b = sum_col4(dlnb[o]);
      if constexpr (RS) {
#pragma unroll
        for (int v = 0; v < NW; ++v) {
          w += red[v * 64 + 16 * o + n];
          b += red[(NW + v) * 64 + 16 * o + n];
        }
      }
      if (g == 0) {
        p.db2[(size_t)chain * F + 16 * o + n] = db2[o];
        p.dln_w[(size_t)chain * F + 16 * o + n] = w;
        p.dln_b[(size_t)chain * F + 16 * o + n] = b;
      }
    }
  }
}

// dXQ = (dout + dA1 XK) + dZ1b W1_s^T and dXK = (-dtgt + dA1^T XQ - e G1 dW1'^T)
// + dZ1 W1_s^T for every mini-batch s, the bracketed terms from the reverse
// sweep's handoff.  One wave per (chain, checkpoint group, feature tile c):
// W1_s^T[:, c] (FF/16 tiles [16 hidden x 16 features]) starts from the group's
// checkpoint and steps forward with the saved update operands,
// W1_{s+1}^T = W1_s^T + (-e G1_s)^T XK_s.  With `poison` (a fused worker
// that gave up waiting for the group) the group's rows get NaN instead.
template <typename T, int FT, int NW, int HT>
__device__ __forceinline__ void mlp_bwd_dx_body(const MlpBwdParams& p, int chain, int kk, bool poison) {
  constexpr int F = 16 * FT;
  constexpr int K = 16;
  constexpr int FF = 16 * HT * NW;
  constexpr int HB = FF / 16;  // hidden blocks
  constexpr int ST = (int)sizeof(T);
  using Slot = MlpSavedSlot<F, FF, ST>;
  using WS = MlpBwdWsSlot<F, FF, ST>;
  const int NC = p.NC, G = p.G, NK = p.NK;
  const int c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // feature tile
  const int l = lane_id(), g = l >> 4, n = l & 15;

  const size_t xoff = (size_t)chain * NC * K * F;
  const unsigned xbytes = (unsigned)((size_t)NC * K * F * ST);
  const rsrc_t rXK = make_rsrc(static_cast<const T*>(p.XK) + xoff, xbytes);
  const rsrc_t rDXQ = make_rsrc(static_cast<T*>(p.dXQ) + xoff, xbytes);
  const rsrc_t rDXK = make_rsrc(static_cast<T*>(p.dXK) + xoff, xbytes);
  const rsrc_t rSV = make_rsrc(static_cast<const char*>(p.saved) + (size_t)chain * NC * Slot::BYTES,
                               (unsigned)(NC * Slot::BYTES));
  const rsrc_t rWS = make_rsrc(static_cast<const char*>(p.ws) + (size_t)chain * NC * WS::BYTES,
                               (unsigned)(NC * WS::BYTES));
  const int xcl = (4 * g * F + n) * ST + 16 * c * ST;  // C-layout tile of feature tile c in a [16 x F] block
  const int hl = l * 4 * ST;                           // + hb * 256 * ST: hidden block hb, lane order
  const int f4l = l * 16 + c * 1024;                   // fp32 tile c, lane order
  const int s0 = kk * G, s1 = min(s0 + G, NC);
  if (poison) {
    const float qnan = __builtin_nanf("");
    const Frag<T> bad = to_frag<T>(f4{qnan, qnan, qnan, qnan});
    for (int s = s0; s < s1; ++s) {
      bstore_ctile<T>(rDXQ, xcl, s * K * F * ST, F, bad);
      bstore_ctile<T>(rDXK, xcl, s * K * F * ST, F, bad);
    }
    return;
  }

  // W1^T tiles [hidden block hb x feature tile c]: lane (g, n) holds
  // W1[16c + n][16 hb + 4g + j], one 16-byte read per tile from the [F][FF] checkpoint
  Tile w[HB];
  {
    const rsrc_t rW1c = make_rsrc(p.W1_ckpt + (size_t)chain * NK * F * FF, (unsigned)((size_t)NK * F * FF * 4));
    const int wl = ((16 * c + n) * FF + 4 * g) * 4;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) w[hb].v = bload_frag<float>(rW1c, wl + hb * 64, kk * F * FF * 4).v;
  }
  // per mini-batch inputs, requested one mini-batch ahead
  struct In {
    f4 aq, ak;
    Frag<T> zb[HB], zk[HB];
  };
  auto load_in = [&](int s, In& in) {
    const int ws_ = s * WS::BYTES;
    in.aq = bload_frag_dev<float>(rWS, f4l, ws_ + WS::XQP).v;
    in.ak = bload_frag_dev<float>(rWS, f4l, ws_ + WS::XKP).v;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      in.zb[hb] = bload_frag_dev<T>(rWS, hl + hb * 256 * ST, ws_ + WS::DZ1BF);
      in.zk[hb] = bload_frag_dev<T>(rWS, hl + hb * 256 * ST, ws_ + WS::DZ1F);
    }
  };
  In cur;
  load_in(s0, cur);
  // retire the loads issued so far: pending on loop entry, they make the
  // wait-count pass wait for every outstanding access in each iteration
  __builtin_amdgcn_s_waitcnt(0);
  for (int s = s0; s < s1; ++s) {
    const int us = s * Slot::BYTES, xo = s * K * F * ST;
    In nxt;
    load_in(s + 1 < s1 ? s + 1 : s, nxt);
    Frag<T> g1e[HB];
    Frag<T> xkT;
    const bool step = s + 1 < s1;
    if (step) {
      xkT = bload_ctile<T>(rXK, xcl, xo, F);  // XK^T frag of feature tile c
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) g1e[hb] = bload_frag<T>(rSV, hl + hb * 256 * ST, us + Slot::G1E);
    }
    f4 aq = cur.aq, ak = cur.ak;
#pragma unroll
    for (int hb = 0; hb < HB; hb += 2) {
      const Frag<T> w0 = to_frag<T>(w[hb].v), w1 = to_frag<T>(w[hb + 1].v);
      mma32(aq, cur.zb[hb], cur.zb[hb + 1], w0, w1);
      mma32(ak, cur.zk[hb], cur.zk[hb + 1], w0, w1);
    }
    bstore_ctile<T>(rDXQ, xcl, xo, F, to_frag<T>(aq));
    bstore_ctile<T>(rDXK, xcl, xo, F, to_frag<T>(ak));
    if (step) {
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) mma16(w[hb].v, g1e[hb], xkT);
    }
    cur = nxt;
  }
}

template <typename T, int FT, int NW, int HT>
__global__ __launch_bounds__(64 * FT) void mlp_bwd_dx_kernel(MlpBwdParams p) {
  const int chain = blockIdx.x / p.NK, kk = blockIdx.x - chain * p.NK;
  mlp_bwd_dx_body<T, FT, NW, HT>(p, chain, kk, false);
}

__global__ void mlp_bwd_ctrl_clear_kernel(int* ctrl, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) ctrl[i] = 0;
}

// compute units of the current device (cached per device)
static int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = v;
  }
  return cus[dev];
}

// Fused when the workgroups are alike (as many sweep waves as feature tiles)
// and every chain's sweep fits on the device at once with CUs to spare for
// workers; otherwise the dXQ/dXK pass is a second launch.
// The control words are cleared in both modes, so that the timeout word read
// by ttt_mlp_bwd_check always belongs to this call.
template <typename T, int FT, int NW, int HT, bool LR, typename ET = T>
static hipError_t launch_mlp_bwd_t(MlpBwdParams p, hipStream_t stream) {
  const int chains = p.B * p.H, cus = device_cus();
  const bool fused = NW == FT && p.dx_fused != 0 && p.dx_ctrl != nullptr && cus >= chains + 16;
  const int nctrl = fused ? kDxCtrlHead + chains * p.NK : kDxCtrlHead;
  hipLaunchKernelGGL(mlp_bwd_ctrl_clear_kernel, dim3((nctrl + 255) / 256), dim3(256), 0, stream, p.dx_ctrl, nctrl);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (!fused) {
    p.dx_ctrl = nullptr;
    hipLaunchKernelGGL((mlp_bwd_kernel<T, FT, NW, HT, LR, ET>), dim3(chains), dim3(64 * NW), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((mlp_bwd_dx_kernel<T, FT, NW, HT>), dim3(chains * p.NK), dim3(64 * FT), 0, stream, p);
    return hipGetLastError();
  }
  // the sweeps, then one worker per CU: the first cus - chains run beside the
  // sweeps, the rest start on the CUs the sweeps leave
  hipLaunchKernelGGL((mlp_bwd_kernel<T, FT, NW, HT, LR, ET>), dim3(chains + cus), dim3(64 * NW), 0, stream, p);
  return hipGetLastError();
}

template <typename T, int FT, int NW, int HT>
static hipError_t launch_mlp_bwd_e(const MlpBwdParams& p, hipStream_t stream) {
  if (p.eta_rule == TTT_ETA_DENSE) return launch_mlp_bwd_t<T, FT, NW, HT, false>(p, stream);
  if (p.eta_rule == TTT_ETA_DENSE_F32) return launch_mlp_bwd_t<T, FT, NW, HT, false, float>(p, stream);
  return launch_mlp_bwd_t<T, FT, NW, HT, true>(p, stream);
}

template <typename T, int FT>
static hipError_t launch_mlp_bwd_f(const MlpBwdParams& p, hipStream_t stream) {
  switch (p.FF) {
    case 64:  // at F = 64 four waves of FF/64 hidden tiles, so that the LayerNorms split by rows
      if constexpr (FT == 4) return launch_mlp_bwd_e<T, FT, 4, 1>(p, stream);
      else return launch_mlp_bwd_e<T, FT, 1, 4>(p, stream);
    case 128:
      if constexpr (FT == 4) return launch_mlp_bwd_e<T, FT, 4, 2>(p, stream);
      else return launch_mlp_bwd_e<T, FT, 2, 4>(p, stream);
    case 256: return launch_mlp_bwd_e<T, FT, 4, 4>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_mlp_bwd(const MlpBwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == TTT_DTYPE_BF16) {
    if (p.F == 64) return launch_mlp_bwd_f<__bf16, 4>(p, stream);
    if (p.F == 32) return launch_mlp_bwd_f<__bf16, 2>(p, stream);
  } else if (dtype == TTT_DTYPE_F16) {
    if (p.F == 64) return launch_mlp_bwd_f<_Float16, 4>(p, stream);
    if (p.F == 32) return launch_mlp_bwd_f<_Float16, 2>(p, stream);
  } else {
    if (p.F == 64) return launch_mlp_bwd_f<float, 4>(p, stream);
    if (p.F == 32) return launch_mlp_bwd_f<float, 2>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ttt
