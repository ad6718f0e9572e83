// extern "C" entry points of libttt_amd.so: host-side validation, then one
// launch per call on the caller's stream.  Declarations and argument
// contracts are in include/ttt_amd.h.
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "ttt_kernels.h"

namespace {

// activation dtypes the kernels take: fp32, bf16, fp16
inline bool dtype_ok(int dtype) {
  return dtype == TTT_DTYPE_F32 || dtype == TTT_DTYPE_BF16 || dtype == TTT_DTYPE_F16;
}

// process-wide options (ttt_set_option)
std::atomic<long long> g_mlp_bwd_poll_limit{1LL << 22};
std::atomic<long long> g_mlp_bwd_fused{1};
std::atomic<long long> g_small_kernels{1};

bool eta_rule_ok(int r) {
  return r == TTT_ETA_DENSE || r == TTT_ETA_LAYER || r == TTT_ETA_CAUSAL || r == TTT_ETA_DENSE_F32;
}
// fp32 dense eta under fp32 activations is the plain dense form
int eta_rule_of(int r, int dtype) { return r == TTT_ETA_DENSE_F32 && dtype == TTT_DTYPE_F32 ? TTT_ETA_DENSE : r; }

// Scratch of ttt_mlp_bwd_noalloc: the backward's workspace (the reverse
// sweep's per-mini-batch handoff and the dXQ/dXK workers' control words) in a
// file-scope device array instead of caller or library allocations.  Each GPU
// holds its own copy for the life of the process; its device address is taken
// once per device with hipGetSymbolAddress (the array's name in host code is
// only a stand-in, never a device address) and used for every launch.
static __device__ __align__(256) unsigned char scratch[TTT_MLP_BWD_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// device address of the current device's scratch, looked up on first use
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TTT_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return TTT_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TTT_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(int B, int H, int NC, int K, int F, int G, int dtype, float eps) {
  if (!dtype_ok(dtype)) return TTT_ERR_DTYPE;
  if (B <= 0 || H <= 0 || NC <= 0) return TTT_ERR_SHAPE;
  if (K < 16 || K > 64 || K % 16 != 0) return TTT_ERR_SHAPE;
  if (F < 16 || F > 256 || F % 16 != 0) return TTT_ERR_SHAPE;
  if (G < 1 || G > NC) return TTT_ERR_ARG;
  if (!(eps > 0.0f) || eps > 1.0f) return TTT_ERR_ARG;
  if ((long long)B * H > 0x7fffffffLL) return TTT_ERR_SHAPE;
  return TTT_OK;
}

#define REQUIRE_PTR(p)                 \
  do {                                 \
    if ((p) == nullptr) return TTT_ERR_NULL; \
    if (!aligned16(p)) return TTT_ERR_ALIGN; \
  } while (0)

#define OPTIONAL_PTR(p)                            \
  do {                                             \
    if ((p) != nullptr && !aligned16(p)) return TTT_ERR_ALIGN; \
  } while (0)

int hip_status(hipError_t e) { return e == hipSuccess ? TTT_OK : TTT_ERR_HIP; }

// Shapes of the specialised inner-loop kernels (16-token mini-batches held in
// registers); every other valid shape takes the general-shape kernels.
bool fast_linear_shape(int K, int F) { return K == 16 && (F == 32 || F == 64); }
bool fast_mlp_shape(int K, int F, int FF) {
  return fast_linear_shape(K, F) && (FF == 64 || FF == 128 || FF == 256);
}
// the fixed-weight kernels (readout, memo combiner): any K, F in {32, 64}
bool fixed_mlp_shape(int F, int FF) { return (F == 32 || F == 64) && (FF == 32 || FF == 64 || FF == 128 || FF == 256); }

// TTT-MLP shapes: hidden width, and per-chain slabs addressable with 32-bit
// byte offsets (the state checkpoints are the largest, NC * F * FF * 4 bytes)
int check_mlp(int NC, int F, int FF, int dtype) {
  if (FF != 64 && FF != 128 && FF != 256) return TTT_ERR_SHAPE;
  if ((long long)NC * F * FF * 4 > 0x7fffffffLL) return TTT_ERR_SHAPE;
  if ((long long)NC * ttt::mlp_saved_slot_bytes(F, FF, dtype) > 0x7fffffffLL) return TTT_ERR_SHAPE;
  return TTT_OK;
}

// TTT-Linear: per-chain saved slots addressed with 32-bit byte offsets
int check_linear(int NC, int F) {
  if ((long long)NC * ttt::linear_saved_slot_bytes(F) > 0x7fffffffLL) return TTT_ERR_SHAPE;
  return TTT_OK;
}

}  // namespace

namespace ttt {
bool gen_force_general() { return g_small_kernels.load() == 0; }
}  // namespace ttt

extern "C" {

int ttt_abi_version(void) { return TTT_AMD_ABI_VERSION; }

const char* ttt_error_string(int status) {
  switch (status) {
    case TTT_OK: return "ok";
    case TTT_ERR_SHAPE: return "unsupported or inconsistent shape";
    case TTT_ERR_DTYPE: return "unsupported dtype";
    case TTT_ERR_NULL: return "required pointer is NULL";
    case TTT_ERR_ALIGN: return "pointer is not 16-byte aligned";
    case TTT_ERR_HIP: return "HIP launch failed";
    case TTT_ERR_WORKSPACE: return "workspace missing or too small";
    case TTT_ERR_ARG: return "invalid argument";
    case TTT_ERR_TIMEOUT: return "a fused dXQ/dXK worker gave up waiting (its rows hold NaN)";
    case TTT_ERR_SCRATCH: return "the problem needs more workspace than the no-allocation entry point's static scratch";
    default: return "unknown status";
  }
}

size_t ttt_linear_saved_bytes(int B, int H, int NC, int K, int F) {
  if (B <= 0 || H <= 0 || NC <= 0) return 0;
  if (fast_linear_shape(K, F)) return (size_t)B * H * NC * ttt::linear_saved_slot_bytes(F);
  if (ttt::gen_shape_ok(K, F, F, false)) return ttt::gen_saved_bytes(B, H, NC, K, F, F, false);
  return 0;
}

int ttt_linear_fwd(const void* XQ, const void* XK, const void* XV, const void* eta, const float* ln_w,
                   const float* ln_b, const float* W1_init, const float* b1_init, int B, int H, int NC, int K,
                   int F, int G, int dtype, int eta_rule, float eps, void* out, float* W1_last, float* b1_last,
                   float* W1_ckpt, float* b1_ckpt, void* saved, size_t saved_bytes, void* stream) {
  int st = check_common(B, H, NC, K, F, G, dtype, eps);
  if (st != TTT_OK) return st;
  if (!eta_rule_ok(eta_rule)) return TTT_ERR_ARG;
  eta_rule = eta_rule_of(eta_rule, dtype);
  st = fast_linear_shape(K, F) ? check_linear(NC, F) : TTT_OK;
  if (st != TTT_OK) return st;
  REQUIRE_PTR(XQ);
  REQUIRE_PTR(XK);
  REQUIRE_PTR(XV);
  REQUIRE_PTR(eta);
  REQUIRE_PTR(ln_w);
  REQUIRE_PTR(ln_b);
  REQUIRE_PTR(W1_init);
  REQUIRE_PTR(b1_init);
  REQUIRE_PTR(out);
  OPTIONAL_PTR(W1_last);
  OPTIONAL_PTR(b1_last);
  OPTIONAL_PTR(W1_ckpt);
  OPTIONAL_PTR(b1_ckpt);
  if ((W1_last == nullptr) != (b1_last == nullptr)) return TTT_ERR_NULL;
  if ((W1_ckpt == nullptr) != (b1_ckpt == nullptr)) return TTT_ERR_NULL;
  if (saved != nullptr) {
    if (!aligned16(saved)) return TTT_ERR_ALIGN;
    if (saved_bytes < ttt_linear_saved_bytes(B, H, NC, K, F)) return TTT_ERR_WORKSPACE;
  }
  if (!fast_linear_shape(K, F)) {
    if (saved == nullptr) return TTT_ERR_WORKSPACE;  // the general path's states and scratch
    ttt::GenFwdParams q{};
    q.XQ = XQ;
    q.XK = XK;
    q.XV = XV;
    q.eta = eta;
    q.ln_w = ln_w;
    q.ln_b = ln_b;
    q.W1_init = W1_init;
    q.b1_init = b1_init;
    q.out = out;
    q.W1_last = W1_last;
    q.b1_last = b1_last;
    q.W1_ckpt = W1_ckpt;
    q.b1_ckpt = b1_ckpt;
    q.saved = saved;
    q.B = B;
    q.H = H;
    q.NC = NC;
    q.K = K;
    q.F = F;
    q.FF = F;
    q.G = G;
    q.M = 1;
    q.eta_rule = eta_rule;
    q.mlp = false;
    q.eps = eps;
    return hip_status(ttt::launch_gen_fwd(q, dtype, static_cast<hipStream_t>(stream)));
  }

  ttt::LinearFwdParams p;
  p.XQ = XQ;
  p.XK = XK;
  p.XV = XV;
  p.eta = eta;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.W_init = W1_init;
  p.b_init = b1_init;
  p.out = out;
  p.W_last = W1_last;
  p.b_last = b1_last;
  p.W_ckpt = W1_ckpt;
  p.b_ckpt = b1_ckpt;
  p.saved = saved;
  p.B = B;
  p.H = H;
  p.NC = NC;
  p.F = F;
  p.G = G;
  p.NK = (NC + G - 1) / G;
  p.eta_rule = eta_rule;
  p.eps = eps;
  return hip_status(ttt::launch_linear_fwd(p, dtype, static_cast<hipStream_t>(stream)));
}

int ttt_linear_bwd(const void* XQ, const void* XK, const void* XV, const void* eta, const float* ln_w,
                   const float* ln_b, const float* W1_ckpt, const float* W1_last, const void* dout, int B, int H,
                   int NC, int K, int F, int G, int dtype, int eta_rule, float eps, void* dXQ, void* dXK,
                   void* dXV, void* deta, float* dW1, float* db1, float* dln_w, float* dln_b, const void* saved,
                   size_t saved_bytes, void* stream) {
  int st = check_common(B, H, NC, K, F, G, dtype, eps);
  if (st != TTT_OK) return st;
  if (!eta_rule_ok(eta_rule)) return TTT_ERR_ARG;
  eta_rule = eta_rule_of(eta_rule, dtype);
  st = fast_linear_shape(K, F) ? check_linear(NC, F) : TTT_OK;
  if (st != TTT_OK) return st;
  REQUIRE_PTR(XQ);
  REQUIRE_PTR(XK);
  REQUIRE_PTR(XV);
  REQUIRE_PTR(eta);
  REQUIRE_PTR(ln_w);
  REQUIRE_PTR(ln_b);
  REQUIRE_PTR(W1_ckpt);
  REQUIRE_PTR(W1_last);
  REQUIRE_PTR(dout);
  REQUIRE_PTR(dXQ);
  REQUIRE_PTR(dXK);
  REQUIRE_PTR(dXV);
  REQUIRE_PTR(deta);
  REQUIRE_PTR(dW1);
  REQUIRE_PTR(db1);
  REQUIRE_PTR(dln_w);
  REQUIRE_PTR(dln_b);
  if (saved == nullptr) return TTT_ERR_WORKSPACE;
  if (!aligned16(saved)) return TTT_ERR_ALIGN;
  if (saved_bytes < ttt_linear_saved_bytes(B, H, NC, K, F)) return TTT_ERR_WORKSPACE;
  if (!fast_linear_shape(K, F)) {
    ttt::GenBwdParams q{};
    q.XQ = XQ;
    q.XK = XK;
    q.XV = XV;
    q.eta = eta;
    q.dout = dout;
    q.ln_w = ln_w;
    q.ln_b = ln_b;
    q.dXQ = dXQ;
    q.dXK = dXK;
    q.dXV = dXV;
    q.deta = deta;
    q.dW1 = dW1;
    q.db1 = db1;
    q.dln_w = dln_w;
    q.dln_b = dln_b;
    q.saved = const_cast<void*>(saved);
    q.B = B;
    q.H = H;
    q.NC = NC;
    q.K = K;
    q.F = F;
    q.FF = F;
    q.eta_rule = eta_rule;
    q.mlp = false;
    q.eps = eps;
    return hip_status(ttt::launch_gen_bwd(q, dtype, static_cast<hipStream_t>(stream)));
  }

  ttt::LinearBwdParams p;
  p.XQ = XQ;
  p.XK = XK;
  p.XV = XV;
  p.eta = eta;
  p.dout = dout;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.W_ckpt = W1_ckpt;
  p.W_last = W1_last;
  p.saved = saved;
  p.dXQ = dXQ;
  p.dXK = dXK;
  p.dXV = dXV;
  p.deta = deta;
  p.dW = dW1;
  p.db = db1;
  p.dln_w = dln_w;
  p.dln_b = dln_b;
  p.B = B;
  p.H = H;
  p.NC = NC;
  p.F = F;
  p.G = G;
  p.NK = (NC + G - 1) / G;
  p.eta_rule = eta_rule;
  return hip_status(ttt::launch_linear_bwd(p, dtype, static_cast<hipStream_t>(stream)));
}

int ttt_mlp_fwd(const void* XQ, const void* XK, const void* XV, const void* eta, const float* ln_w,
                const float* ln_b, const float* W1_init, const float* b1_init, const float* W2_init,
                const float* b2_init, int B, int H, int NC, int K, int F, int FF, int G, int M, int dtype,
                int eta_rule, float eps, void* out, float* W1_last, float* b1_last, float* W2_last, float* b2_last, float* W1_ckpt,
                float* b1_ckpt, float* W2_ckpt, float* b2_ckpt, float* W1_memo, float* b1_memo, float* W2_memo,
                float* b2_memo, void* saved, size_t saved_bytes, void* stream) {
  int st = check_common(B, H, NC, K, F, G, dtype, eps);
  if (st != TTT_OK) return st;
  const bool fast = fast_mlp_shape(K, F, FF);
  if (!fast && !ttt::gen_shape_ok(K, F, FF, true)) return TTT_ERR_SHAPE;
  st = fast ? check_mlp(NC, F, FF, dtype) : TTT_OK;
  if (st != TTT_OK) return st;
  if (!eta_rule_ok(eta_rule)) return TTT_ERR_ARG;
  eta_rule = eta_rule_of(eta_rule, dtype);
  REQUIRE_PTR(XQ);
  REQUIRE_PTR(XK);
  REQUIRE_PTR(XV);
  REQUIRE_PTR(eta);
  REQUIRE_PTR(ln_w);
  REQUIRE_PTR(ln_b);
  REQUIRE_PTR(W1_init);
  REQUIRE_PTR(b1_init);
  REQUIRE_PTR(W2_init);
  REQUIRE_PTR(b2_init);
  REQUIRE_PTR(out);
  const float* groups[2][4] = {{W1_last, b1_last, W2_last, b2_last}, {W1_memo, b1_memo, W2_memo, b2_memo}};
  for (auto& grp : groups) {
    const bool any = grp[0] || grp[1] || grp[2] || grp[3];
    const bool all = grp[0] && grp[1] && grp[2] && grp[3];
    if (any && !all) return TTT_ERR_NULL;
    for (const float* q : grp) OPTIONAL_PTR(q);
  }
  // checkpoints: W1's, and any of the other three beside it
  if (W1_ckpt == nullptr && (b1_ckpt || W2_ckpt || b2_ckpt)) return TTT_ERR_NULL;
  for (const float* q : {W1_ckpt, b1_ckpt, W2_ckpt, b2_ckpt}) OPTIONAL_PTR(q);
  if (W1_memo != nullptr && M < 1) return TTT_ERR_ARG;
  if (saved != nullptr) {
    if (!aligned16(saved)) return TTT_ERR_ALIGN;
    if (saved_bytes < ttt_mlp_saved_bytes(B, H, NC, K, F, FF, dtype)) return TTT_ERR_WORKSPACE;
  }
  if (!fast) {
    if (saved == nullptr) return TTT_ERR_WORKSPACE;  // the general path's states and scratch
    ttt::GenFwdParams q{};
    q.XQ = XQ;
    q.XK = XK;
    q.XV = XV;
    q.eta = eta;
    q.ln_w = ln_w;
    q.ln_b = ln_b;
    q.W1_init = W1_init;
    q.b1_init = b1_init;
    q.W2_init = W2_init;
    q.b2_init = b2_init;
    q.out = out;
    q.W1_last = W1_last;
    q.b1_last = b1_last;
    q.W2_last = W2_last;
    q.b2_last = b2_last;
    q.W1_ckpt = W1_ckpt;
    q.b1_ckpt = b1_ckpt;
    q.W2_ckpt = W2_ckpt;
    q.b2_ckpt = b2_ckpt;
    q.W1_memo = W1_memo;
    q.b1_memo = b1_memo;
    q.W2_memo = W2_memo;
    q.b2_memo = b2_memo;
    q.saved = saved;
    q.B = B;
    q.H = H;
    q.NC = NC;
    q.K = K;
    q.F = F;
    q.FF = FF;
    q.G = G;
    q.M = W1_memo != nullptr ? M : 1;
    q.eta_rule = eta_rule;
    q.mlp = true;
    q.eps = eps;
    return hip_status(ttt::launch_gen_fwd(q, dtype, static_cast<hipStream_t>(stream)));
  }

  ttt::MlpFwdParams p;
  p.XQ = XQ;
  p.XK = XK;
  p.XV = XV;
  p.eta = eta;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.W1_init = W1_init;
  p.b1_init = b1_init;
  p.W2_init = W2_init;
  p.b2_init = b2_init;
  p.out = out;
  p.W1_last = W1_last;
  p.b1_last = b1_last;
  p.W2_last = W2_last;
  p.b2_last = b2_last;
  p.W1_ckpt = W1_ckpt;
  p.b1_ckpt = b1_ckpt;
  p.W2_ckpt = W2_ckpt;
  p.b2_ckpt = b2_ckpt;
  p.W1_memo = W1_memo;
  p.b1_memo = b1_memo;
  p.W2_memo = W2_memo;
  p.b2_memo = b2_memo;
  p.saved = saved;
  p.B = B;
  p.H = H;
  p.NC = NC;
  p.F = F;
  p.FF = FF;
  p.G = G;
  p.NK = (NC + G - 1) / G;
  p.M = W1_memo != nullptr ? M : 1;
  p.NS = (NC + p.M - 1) / p.M;
  p.eta_rule = eta_rule;
  p.eps = eps;
  return hip_status(ttt::launch_mlp_fwd(p, dtype, static_cast<hipStream_t>(stream)));
}

size_t ttt_mlp_saved_bytes(int B, int H, int NC, int K, int F, int FF, int dtype) {
  if (B <= 0 || H <= 0 || NC <= 0 || K <= 0 || F <= 0 || FF <= 0) return 0;
  if (!dtype_ok(dtype)) return 0;
  if (fast_mlp_shape(K, F, FF)) return (size_t)B * H * NC * ttt::mlp_saved_slot_bytes(F, FF, dtype);
  if (ttt::gen_shape_ok(K, F, FF, true)) return ttt::gen_saved_bytes(B, H, NC, K, F, FF, true);
  return 0;
}

size_t ttt_mlp_bwd_workspace_bytes(int B, int H, int NC, int K, int F, int FF, int dtype) {
  if (B <= 0 || H <= 0 || NC <= 0 || K <= 0 || F <= 0 || FF <= 0) return 0;
  if (!dtype_ok(dtype)) return 0;
  if (fast_mlp_shape(K, F, FF))
    return (size_t)B * H * NC * ttt::mlp_bwd_ws_slot_bytes(F, FF, dtype) + ttt::mlp_bwd_ctrl_bytes(B, H, NC, 1);
  if (ttt::small_shape_ok(K, F, FF, true)) {
    // the register-resident kernels' handoff (they also run with the minimum, in one launch)
    const size_t hb = ttt::small_mlp_bwd_hand_bytes(B, H, NC, K);
    return hb > 256 ? hb : 256;
  }
  if (ttt::gen_shape_ok(K, F, FF, true)) return 256;  // (the general path keeps its scratch in `saved`)
  return 0;
}

namespace {
// the least workspace the MLP backward runs with: the whole for the
// specialised kernels, 256 bytes for the rest
size_t mlp_bwd_min_workspace(int B, int H, int NC, int K, int F, int FF, int dtype) {
  const size_t need = ttt_mlp_bwd_workspace_bytes(B, H, NC, K, F, FF, dtype);
  return fast_mlp_shape(K, F, FF) || need == 0 ? need : 256;
}
}  // namespace

static int mlp_bwd_impl(const void* XQ, const void* XK, const void* XV, const void* eta, const float* ln_w,
                const float* ln_b, const float* W1_ckpt, const float* b1_ckpt, const float* W2_ckpt,
                const float* b2_ckpt, const float* W1_last, const float* b1_last, const float* W2_last,
                const float* b2_last, const void* dout, int B, int H, int NC, int K, int F, int FF, int G, int dtype,
                int eta_rule, float eps, void* dXQ, void* dXK, void* dXV, void* deta, float* dW1, float* db1, float* dW2,
                float* db2, float* dln_w, float* dln_b, const void* saved, size_t saved_bytes, void* workspace,
                size_t workspace_bytes, void* stream) {
  int st = check_common(B, H, NC, K, F, G, dtype, eps);
  if (st != TTT_OK) return st;
  const bool fast = fast_mlp_shape(K, F, FF);
  if (!fast && !ttt::gen_shape_ok(K, F, FF, true)) return TTT_ERR_SHAPE;
  st = fast ? check_mlp(NC, F, FF, dtype) : TTT_OK;
  if (st != TTT_OK) return st;
  if (!eta_rule_ok(eta_rule)) return TTT_ERR_ARG;
  eta_rule = eta_rule_of(eta_rule, dtype);
  (void)b1_ckpt;  // not read: the saved values carry the rest of the state
  (void)W2_ckpt;
  (void)b2_ckpt;
  const void* req[] = {XQ, XK, XV, eta, ln_w, ln_b, W1_ckpt,
                       W1_last, b1_last, W2_last, b2_last, dout,
                       dXQ, dXK, dXV, deta, dW1, db1, dW2, db2, dln_w, dln_b};
  for (const void* q : req) REQUIRE_PTR(q);
  if (saved == nullptr) return TTT_ERR_WORKSPACE;
  if (!aligned16(saved)) return TTT_ERR_ALIGN;
  if (saved_bytes < ttt_mlp_saved_bytes(B, H, NC, K, F, FF, dtype)) return TTT_ERR_WORKSPACE;
  if (workspace == nullptr) return TTT_ERR_WORKSPACE;
  if (!aligned16(workspace)) return TTT_ERR_ALIGN;
  if (workspace_bytes < mlp_bwd_min_workspace(B, H, NC, K, F, FF, dtype)) return TTT_ERR_WORKSPACE;
  if (!fast) {
    ttt::GenBwdParams q{};
    q.ws = workspace;
    q.ws_bytes = workspace_bytes;
    q.XQ = XQ;
    q.XK = XK;
    q.XV = XV;
    q.eta = eta;
    q.dout = dout;
    q.ln_w = ln_w;
    q.ln_b = ln_b;
    q.dXQ = dXQ;
    q.dXK = dXK;
    q.dXV = dXV;
    q.deta = deta;
    q.dW1 = dW1;
    q.db1 = db1;
    q.dW2 = dW2;
    q.db2 = db2;
    q.dln_w = dln_w;
    q.dln_b = dln_b;
    q.saved = const_cast<void*>(saved);
    q.B = B;
    q.H = H;
    q.NC = NC;
    q.K = K;
    q.F = F;
    q.FF = FF;
    q.eta_rule = eta_rule;
    q.mlp = true;
    q.eps = eps;
    return hip_status(ttt::launch_gen_bwd(q, dtype, static_cast<hipStream_t>(stream)));
  }

  ttt::MlpBwdParams p;
  p.XQ = XQ;
  p.XK = XK;
  p.XV = XV;
  p.eta = eta;
  p.dout = dout;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.W1_ckpt = W1_ckpt;
  p.b1_ckpt = b1_ckpt;
  p.W2_ckpt = W2_ckpt;
  p.b2_ckpt = b2_ckpt;
  p.W1_last = W1_last;
  p.b1_last = b1_last;
  p.W2_last = W2_last;
  p.b2_last = b2_last;
  p.saved = saved;
  p.ws = workspace;
  // control words behind the handoff slots (sized for G = 1, the most groups)
  p.dx_ctrl = reinterpret_cast<int*>(static_cast<char*>(workspace) +
                                     (size_t)B * H * NC * ttt::mlp_bwd_ws_slot_bytes(F, FF, dtype));
  p.dXQ = dXQ;
  p.dXK = dXK;
  p.dXV = dXV;
  p.deta = deta;
  p.dW1 = dW1;
  p.db1 = db1;
  p.dW2 = dW2;
  p.db2 = db2;
  p.dln_w = dln_w;
  p.dln_b = dln_b;
  p.B = B;
  p.H = H;
  p.NC = NC;
  p.F = F;
  p.FF = FF;
  p.G = G;
  p.NK = (NC + G - 1) / G;
  p.eta_rule = eta_rule;
  p.dx_max_polls = (int)g_mlp_bwd_poll_limit.load();
  p.dx_fused = (int)g_mlp_bwd_fused.load();
  p.eps = eps;
  return hip_status(ttt::launch_mlp_bwd(p, dtype, static_cast<hipStream_t>(stream)));
}

int ttt_mlp_bwd(const void* XQ, const void* XK, const void* XV, const void* eta, const float* ln_w,
                const float* ln_b, const float* W1_ckpt, const float* b1_ckpt, const float* W2_ckpt,
                const float* b2_ckpt, const float* W1_last, const float* b1_last, const float* W2_last,
                const float* b2_last, const void* dout, int B, int H, int NC, int K, int F, int FF, int G, int dtype,
                int eta_rule, float eps, void* dXQ, void* dXK, void* dXV, void* deta, float* dW1, float* db1,
                float* dW2, float* db2, float* dln_w, float* dln_b, const void* saved, size_t saved_bytes,
                void* workspace, size_t workspace_bytes, void* stream) {
  return mlp_bwd_impl(XQ, XK, XV, eta, ln_w, ln_b, W1_ckpt, b1_ckpt, W2_ckpt, b2_ckpt, W1_last, b1_last, W2_last,
                      b2_last, dout, B, H, NC, K, F, FF, G, dtype, eta_rule, eps, dXQ, dXK, dXV, deta, dW1, db1, dW2,
                      db2, dln_w, dln_b, saved, saved_bytes, workspace, workspace_bytes, stream);
}

int ttt_mlp_bwd_noalloc(const void* XQ, const void* XK, const void* XV, const void* eta, const float* ln_w,
                        const float* ln_b, const float* W1_ckpt, const float* b1_ckpt, const float* W2_ckpt,
                        const float* b2_ckpt, const float* W1_last, const float* b1_last, const float* W2_last,
                        const float* b2_last, const void* dout, int B, int H, int NC, int K, int F, int FF, int G,
                        int dtype, int eta_rule, float eps, void* dXQ, void* dXK, void* dXV, void* deta, float* dW1,
                        float* db1, float* dW2, float* db2, float* dln_w, float* dln_b, const void* saved,
                        size_t saved_bytes, void* stream) {
  // (the register-resident kernels take the two-launch form when their
  // handoff fits the scratch, else the one-launch form)
  const size_t need = mlp_bwd_min_workspace(B, H, NC, K, F, FF, dtype);
  if (need == 0) return !dtype_ok(dtype) ? TTT_ERR_DTYPE : TTT_ERR_SHAPE;
  if (need > TTT_MLP_BWD_NOALLOC_SCRATCH_BYTES) return TTT_ERR_SCRATCH;
  void* ws = nullptr;
  const int st = scratch_of_current_device(&ws);
  if (st != TTT_OK) return st;
  // the launch clears the control words it uses with a fill kernel; the
  // handoff slots are written before they are read
  return mlp_bwd_impl(XQ, XK, XV, eta, ln_w, ln_b, W1_ckpt, b1_ckpt, W2_ckpt, b2_ckpt, W1_last, b1_last, W2_last,
                      b2_last, dout, B, H, NC, K, F, FF, G, dtype, eta_rule, eps, dXQ, dXK, dXV, deta, dW1, db1, dW2,
                      db2, dln_w, dln_b, saved, saved_bytes, ws, TTT_MLP_BWD_NOALLOC_SCRATCH_BYTES, stream);
}

int ttt_set_option(int option, long long value) {
  switch (option) {
    case TTT_OPT_MLP_BWD_POLL_LIMIT:
      if (value < 0 || value > 0x7fffffffLL) return TTT_ERR_ARG;
      g_mlp_bwd_poll_limit.store(value);
      return TTT_OK;
    case TTT_OPT_MLP_BWD_FUSED:
      if (value != 0 && value != 1) return TTT_ERR_ARG;
      g_mlp_bwd_fused.store(value);
      return TTT_OK;
    case TTT_OPT_SMALL_KERNELS:
      if (value != 0 && value != 1) return TTT_ERR_ARG;
      g_small_kernels.store(value);
      return TTT_OK;
    default: return TTT_ERR_ARG;
  }
}

long long ttt_get_option(int option) {
  switch (option) {
    case TTT_OPT_MLP_BWD_POLL_LIMIT: return g_mlp_bwd_poll_limit.load();
    case TTT_OPT_MLP_BWD_FUSED: return g_mlp_bwd_fused.load();
    case TTT_OPT_SMALL_KERNELS: return g_small_kernels.load();
    default: return -1;
  }
}

int ttt_mlp_bwd_check(const void* workspace, size_t workspace_bytes, int B, int H, int NC, int K, int F, int FF,
                      int dtype, void* stream) {
  const size_t need = ttt_mlp_bwd_workspace_bytes(B, H, NC, K, F, FF, dtype);
  if (need == 0) return TTT_ERR_SHAPE;
  if (!fast_mlp_shape(K, F, FF)) return TTT_OK;  // no fused workers, no timeout word
  if (workspace == nullptr) {  // the no-allocation entry point's scratch on the current device
    if (need > TTT_MLP_BWD_NOALLOC_SCRATCH_BYTES) return TTT_ERR_SCRATCH;
    void* ws = nullptr;
    const int st = scratch_of_current_device(&ws);
    if (st != TTT_OK) return st;
    workspace = ws;
    workspace_bytes = TTT_MLP_BWD_NOALLOC_SCRATCH_BYTES;
  }
  if (workspace_bytes < need) return TTT_ERR_WORKSPACE;
  // the timeout word: control word 1 behind the B*H*NC handoff slots
  const int* ctrl = reinterpret_cast<const int*>(static_cast<const char*>(workspace) +
                                                 (size_t)B * H * NC * ttt::mlp_bwd_ws_slot_bytes(F, FF, dtype));
  int word = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(&word, ctrl + 1, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess) return TTT_ERR_HIP;
  if (hipStreamSynchronize(s) != hipSuccess) return TTT_ERR_HIP;
  return word != 0 ? TTT_ERR_TIMEOUT : TTT_OK;
}

int ttt_mlp_cached_readout(const void* XQ, const float* W1, const float* b1, const float* W2, const float* b2,
                           const float* ln_w, const float* ln_b, int B, int H, int NS, int K, int F, int FF, int S,
                           int dtype, float eps, float* out, void* stream) {
  int st = check_common(B, H, NS, K, F, 1, dtype, eps);
  if (st != TTT_OK) return st;
  if (!fixed_mlp_shape(F, FF)) return TTT_ERR_SHAPE;
  if (S < 1) return TTT_ERR_ARG;
  if ((long long)NS * K > 0x7fffffffLL / 64) return TTT_ERR_SHAPE;
  const void* req[] = {XQ, W1, b1, W2, b2, ln_w, ln_b, out};
  for (const void* q : req) REQUIRE_PTR(q);

  ttt::MlpReadoutParams p;
  p.XQ = XQ;
  p.W1 = W1;
  p.b1 = b1;
  p.W2 = W2;
  p.b2 = b2;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.out = out;
  p.B = B;
  p.H = H;
  p.ntok = NS * K;
  p.F = F;
  p.FF = FF;
  p.S = S;
  const int chunk = ttt::mlp_readout_chunk_tokens();
  p.nchunk = (p.ntok + chunk - 1) / chunk;
  if ((long long)B * H * p.nchunk > 0x7fffffffLL) return TTT_ERR_SHAPE;
  p.eps = eps;
  return hip_status(ttt::launch_mlp_readout(p, dtype, static_cast<hipStream_t>(stream)));
}

// The combiner's kernels walk 16-token tiles: a mini-batch of K = 16 k tokens
// is k tiles and a segment of M mini-batches M k tiles (same tokens, same
// segments), so every K is handled as K = 16 with NC k mini-batches.
size_t ttt_mlp_memo_gates_bytes(int B, int H, int NC, int K, int F, int M) {
  if (B <= 0 || H <= 0 || NC <= 0 || K < 16 || K > 64 || K % 16 != 0 || (F != 32 && F != 64) || M < 1) return 0;
  const int k = K / 16;
  return (size_t)B * H * ttt::memo_gate_floats_per_chain(NC * k, 16, F, M * k) * sizeof(float);
}

size_t ttt_mlp_memo_workspace_bytes(int B, int H, int NC, int K, int F, int FF, int M, int dtype) {
  const size_t gb = ttt_mlp_memo_gates_bytes(B, H, NC, K, F, M);
  if (gb == 0 || !fixed_mlp_shape(F, FF) || !dtype_ok(dtype)) return 0;
  if (dtype == TTT_DTYPE_F32) return gb;
  const size_t NS = (size_t)(NC + M - 1) / M;
  return ((gb + 255) & ~(size_t)255) + (size_t)B * H * NS * ttt::mlp_memo_image_bytes(F, FF);
}

namespace {
// the packed memo-state images behind the gates, when the workspace holds them
unsigned char* memo_packed(float* gates, size_t gates_bytes, int B, int H, int NC, int K, int F, int FF, int M,
                           int dtype) {
  if (dtype == TTT_DTYPE_F32) return nullptr;
  const size_t need = ttt_mlp_memo_workspace_bytes(B, H, NC, K, F, FF, M, dtype);
  if (need == 0 || gates_bytes < need) return nullptr;
  return reinterpret_cast<unsigned char*>(gates) + ((ttt_mlp_memo_gates_bytes(B, H, NC, K, F, M) + 255) & ~(size_t)255);
}

int check_memo(int B, int H, int NC, int K, int F, int FF, int M, int dtype, float eps, size_t gates_bytes,
               const float* gates) {
  int st = check_common(B, H, NC, K, F, 1, dtype, eps);
  if (st != TTT_OK) return st;
  if (!fixed_mlp_shape(F, FF)) return TTT_ERR_SHAPE;
  if (M < 1) return TTT_ERR_ARG;
  if ((NC + M - 1) / M > ttt::kMemoMaxStates) return TTT_ERR_SHAPE;
  if ((long long)NC * K * F > 0x7fffffffLL / 4) return TTT_ERR_SHAPE;
  if (gates == nullptr) return TTT_ERR_WORKSPACE;
  if (!aligned16(gates)) return TTT_ERR_ALIGN;
  if (gates_bytes < ttt_mlp_memo_gates_bytes(B, H, NC, K, F, M)) return TTT_ERR_WORKSPACE;
  return TTT_OK;
}

ttt::MlpMemoParams memo_params(const void* XQ, const void* XQW, const float* W1, const float* b1, const float* W2,
                               const float* b2, const float* ln_w, const float* ln_b, int B, int H, int NC, int F,
                               int FF, int M, float eps, float* gates) {
  ttt::MlpMemoParams p{};
  p.XQ = XQ;
  p.XQW = XQW;
  p.W1 = W1;
  p.b1 = b1;
  p.W2 = W2;
  p.b2 = b2;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.gates = gates;
  p.B = B;
  p.H = H;
  p.NC = NC;
  p.F = F;
  p.FF = FF;
  p.M = M;
  p.NS = (NC + M - 1) / M;
  const int ct = ttt::mlp_memo_chunk_tiles(B, H, NC);
  p.nchunk = (NC + ct - 1) / ct;
  p.eps = eps;
  return p;
}
}  // namespace

int ttt_mlp_memo_combine(const void* XQ, const void* XK, const void* XU, const void* XQW, const float* W1_memo,
                         const float* b1_memo, const float* W2_memo, const float* b2_memo, const float* ln_w,
                         const float* ln_b, int B, int H, int NC, int K, int F, int FF, int M, int dtype, float eps,
                         void* out, float* gates, size_t gates_bytes, void* stream) {
  int st = check_memo(B, H, NC, K, F, FF, M, dtype, eps, gates_bytes, gates);
  if (st != TTT_OK) return st;
  const void* req[] = {XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, out};
  for (const void* q : req) REQUIRE_PTR(q);
  const int k = K / 16;  // 16-token tiles per mini-batch
  ttt::MlpMemoParams p = memo_params(XQ, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, B, H, NC * k, F, FF,
                                     M * k, eps, gates);
  p.XK = XK;
  p.XU = XU;
  p.out = out;
  p.packed = memo_packed(gates, gates_bytes, B, H, NC, K, F, FF, M, dtype);
  if ((long long)B * H * p.nchunk > 0x7fffffffLL) return TTT_ERR_SHAPE;
  return hip_status(ttt::launch_mlp_memo(p, dtype, false, static_cast<hipStream_t>(stream)));
}

int ttt_mlp_memo_combine_bwd(const void* XQ, const void* XU, const void* XQW, const float* W1_memo,
                             const float* b1_memo, const float* W2_memo, const float* b2_memo, const float* ln_w,
                             const float* ln_b, const void* dout, int B, int H, int NC, int K, int F, int FF, int M,
                             int dtype, float eps, float* gates, size_t gates_bytes, void* dXK, void* dXU,
                             void* dXQW, void* stream) {
  int st = check_memo(B, H, NC, K, F, FF, M, dtype, eps, gates_bytes, gates);
  if (st != TTT_OK) return st;
  const void* req[] = {XQ, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, dout, dXK, dXU, dXQW};
  for (const void* q : req) REQUIRE_PTR(q);
  const int k = K / 16;  // 16-token tiles per mini-batch
  ttt::MlpMemoParams p = memo_params(XQ, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, B, H, NC * k, F, FF,
                                     M * k, eps, gates);
  p.XU = XU;
  p.dout = dout;
  p.dXK = dXK;
  p.dXU = dXU;
  p.dXQW = dXQW;
  p.packed = memo_packed(gates, gates_bytes, B, H, NC, K, F, FF, M, dtype);
  if ((long long)B * H * p.nchunk > 0x7fffffffLL) return TTT_ERR_SHAPE;
  return hip_status(ttt::launch_mlp_memo(p, dtype, true, static_cast<hipStream_t>(stream)));
}

namespace {
int check_layer_io(int B, int L, int H, int K, int F, int dtype) {
  if (!dtype_ok(dtype)) return TTT_ERR_DTYPE;
  if (B <= 0 || L <= 0 || H <= 0) return TTT_ERR_SHAPE;
  if (K < 16 || K > 64 || K % 16 != 0 || L % K != 0) return TTT_ERR_SHAPE;
  if (F != 32 && F != 64) return TTT_ERR_SHAPE;
  if ((long long)H * F > ttt::layer_io_max_width()) return TTT_ERR_SHAPE;
  if ((long long)B * L > 0x7fffffffLL) return TTT_ERR_SHAPE;
  return TTT_OK;
}
}  // namespace

size_t ttt_layer_io_partial_bytes(int B, int L, int H, int F) {
  if (B <= 0 || L <= 0 || H <= 0 || F <= 0) return 0;
  return (size_t)ttt::layer_io_bwd_blocks(B, L) * 2 * H * F * sizeof(float);
}

int ttt_qkvu_producer_fwd(const void* proj, int ld, const float* rope, const float* ln_w, const float* ln_b, int B,
                          int L, int H, int K, int F, float base_lr, float eps, int dtype, void* XQ, void* XK,
                          void* XV, void* XU, float* lr, void* stream) {
  int st = check_layer_io(B, L, H, K, F, dtype);
  if (st != TTT_OK) return st;
  if (ld < 4 * H * F + H || ld % 4 != 0) return TTT_ERR_SHAPE;
  if (!(eps > 0.0f) || eps > 1.0f) return TTT_ERR_ARG;
  const void* req[] = {proj, rope, ln_w, ln_b, XQ, XK, XV, XU, lr};
  for (const void* q : req) REQUIRE_PTR(q);
  ttt::ProducerParams p{};
  p.proj = proj;
  p.ld = ld;
  p.rope = rope;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.XQ = XQ;
  p.XK = XK;
  p.XV = XV;
  p.XU = XU;
  p.lr = lr;
  p.B = B;
  p.L = L;
  p.H = H;
  p.F = F;
  p.base_lr = base_lr;
  p.eps = eps;
  p.l2eps = 1e-12f;
  return hip_status(ttt::launch_producer(p, dtype, false, static_cast<hipStream_t>(stream)));
}

int ttt_qkvu_producer_bwd(const void* proj, int ld, const float* rope, const float* ln_w, const float* ln_b,
                          const void* dXQ, const void* dXK, const void* dXV, const void* dXU, const float* dlr, int B,
                          int L, int H, int K, int F, float base_lr, float eps, int dtype, void* dproj,
                          float* partial, size_t partial_bytes, void* stream) {
  int st = check_layer_io(B, L, H, K, F, dtype);
  if (st != TTT_OK) return st;
  if (ld < 4 * H * F + H || ld % 4 != 0) return TTT_ERR_SHAPE;
  if (!(eps > 0.0f) || eps > 1.0f) return TTT_ERR_ARG;
  const void* req[] = {proj, rope, ln_w, ln_b, dXQ, dXK, dXV, dXU, dproj};
  for (const void* q : req) REQUIRE_PTR(q);
  OPTIONAL_PTR(dlr);
  if (partial == nullptr) return TTT_ERR_WORKSPACE;
  if (!aligned16(partial)) return TTT_ERR_ALIGN;
  if (partial_bytes < ttt_layer_io_partial_bytes(B, L, H, F)) return TTT_ERR_WORKSPACE;
  ttt::ProducerParams p{};
  p.proj = proj;
  p.ld = ld;
  p.rope = rope;
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.dXQ = dXQ;
  p.dXK = dXK;
  p.dXV = dXV;
  p.dXU = dXU;
  p.dlr = dlr;
  p.dproj = dproj;
  p.partial = partial;
  p.B = B;
  p.L = L;
  p.H = H;
  p.F = F;
  p.base_lr = base_lr;
  p.eps = eps;
  p.l2eps = 1e-12f;
  return hip_status(ttt::launch_producer(p, dtype, true, static_cast<hipStream_t>(stream)));
}

int ttt_post_norm_fwd(const void* XQW, const float* gamma, const float* beta, int B, int L, int H, int K, int F,
                      float eps, int dtype, void* out, float* stats, void* stream) {
  int st = check_layer_io(B, L, H, K, F, dtype);
  if (st != TTT_OK) return st;
  if (!(eps > 0.0f) || eps > 1.0f) return TTT_ERR_ARG;
  const void* req[] = {XQW, gamma, beta, out, stats};
  for (const void* q : req) REQUIRE_PTR(q);
  ttt::PostNormParams p{};
  p.X = XQW;
  p.gamma = gamma;
  p.beta = beta;
  p.Y = out;
  p.stats = stats;
  p.B = B;
  p.L = L;
  p.H = H;
  p.F = F;
  p.eps = eps;
  return hip_status(ttt::launch_post_norm(p, dtype, false, static_cast<hipStream_t>(stream)));
}

int ttt_post_norm_bwd(const void* XQW, const float* gamma, const float* stats, const void* dout, int B, int L, int H,
                      int K, int F, int dtype, void* dXQW, float* partial, size_t partial_bytes, void* stream) {
  int st = check_layer_io(B, L, H, K, F, dtype);
  if (st != TTT_OK) return st;
  const void* req[] = {XQW, gamma, stats, dout, dXQW};
  for (const void* q : req) REQUIRE_PTR(q);
  if (partial == nullptr) return TTT_ERR_WORKSPACE;
  if (!aligned16(partial)) return TTT_ERR_ALIGN;
  if (partial_bytes < ttt_layer_io_partial_bytes(B, L, H, F)) return TTT_ERR_WORKSPACE;
  ttt::PostNormParams p{};
  p.X = XQW;
  p.gamma = gamma;
  p.stats = const_cast<float*>(stats);  // read only in the backward
  p.dY = dout;
  p.dX = dXQW;
  p.partial = partial;
  p.B = B;
  p.L = L;
  p.H = H;
  p.F = F;
  return hip_status(ttt::launch_post_norm(p, dtype, true, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
