"""The C ABI without a GPU: libttt_amd.so loads, exports every function that
include/ttt_amd.h declares (with the argument count the ctypes table uses),
and host-side validation returns the documented status codes.  Every call
below is rejected before any launch, so no device is touched."""

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ttt_amd.h")

OK, E_SHAPE, E_DTYPE, E_NULL, E_ALIGN, E_HIP, E_WS, E_ARG, E_TIMEOUT = 0, -1, -2, -3, -4, -5, -6, -7, -8
F32, BF16, F16 = 0, 1, 2
DENSE, LAYER, CAUSAL = 0, 1, 2
P = 0x10000  # an aligned, never-dereferenced address
Q = 0x10008  # misaligned


def _declarations():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(ttt_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.M | re.S):
        args = [a.strip() for a in m.group(2).split(",") if a.strip()]
        if args == ["void"]:
            args = []
        decls[m.group(1)] = len(args)
    return decls


@pytest.fixture(scope="module")
def lib():
    from ttt_amd import _lib
    return _lib.load()


def test_header_declares_the_abi():
    decls = _declarations()
    for name in ("ttt_abi_version", "ttt_error_string", "ttt_linear_fwd", "ttt_linear_bwd",
                 "ttt_linear_saved_bytes", "ttt_mlp_fwd", "ttt_mlp_bwd", "ttt_mlp_saved_bytes",
                 "ttt_mlp_bwd_workspace_bytes",
                 "ttt_mlp_cached_readout", "ttt_mlp_memo_gates_bytes", "ttt_mlp_memo_workspace_bytes",
                 "ttt_mlp_memo_combine",
                 "ttt_mlp_memo_combine_bwd", "ttt_set_option", "ttt_get_option", "ttt_mlp_bwd_check"):
        assert name in decls, name


def test_every_declared_symbol_is_exported(lib):
    from ttt_amd import _lib
    decls = _declarations()
    assert set(decls) == set(_lib.SIGNATURES), set(decls) ^ set(_lib.SIGNATURES)
    for name, nargs in decls.items():
        assert hasattr(lib, name), name
        assert len(_lib.SIGNATURES[name][1]) == nargs, (name, nargs, len(_lib.SIGNATURES[name][1]))


def test_version_and_error_strings(lib):
    from ttt_amd import _lib
    assert lib.ttt_abi_version() == _lib.ABI_VERSION
    for code in (OK, E_SHAPE, E_DTYPE, E_NULL, E_ALIGN, E_HIP, E_WS, E_ARG, E_TIMEOUT):
        assert lib.ttt_error_string(code)
    assert lib.ttt_error_string(-99) == b"unknown status"


def _lin_fwd(lib, **kw):
    a = dict(XQ=P, XK=P, XV=P, eta=P, lw=P, lb=P, W=P, b=P, B=2, H=4, NC=16, K=16, F=64, G=4, dtype=F32,
             eta_rule=DENSE, eps=1e-8, out=P, Wl=None, bl=None, Wc=None, bc=None, saved=None, saved_bytes=0, stream=None)
    a.update(kw)
    return lib.ttt_linear_fwd(*a.values())


def test_linear_fwd_validation(lib):
    assert _lin_fwd(lib, K=8) == E_SHAPE
    assert _lin_fwd(lib, K=80) == E_SHAPE
    assert _lin_fwd(lib, K=24) == E_SHAPE
    assert _lin_fwd(lib, F=40) == E_SHAPE
    assert _lin_fwd(lib, F=272) == E_SHAPE
    # shapes outside the specialised kernels' set (K = 16, F in {32, 64}) take
    # the general-shape kernels, whose forward needs the saved buffer
    assert _lin_fwd(lib, K=64, F=32) == E_WS
    assert _lin_fwd(lib, K=16, F=48) == E_WS
    assert _lin_fwd(lib, B=0) == E_SHAPE
    assert _lin_fwd(lib, dtype=7) == E_DTYPE
    assert _lin_fwd(lib, XQ=None) == E_NULL
    assert _lin_fwd(lib, out=None) == E_NULL
    assert _lin_fwd(lib, XK=Q) == E_ALIGN
    assert _lin_fwd(lib, G=0) == E_ARG
    assert _lin_fwd(lib, G=17) == E_ARG
    assert _lin_fwd(lib, eps=0.0) == E_ARG
    assert _lin_fwd(lib, eta_rule=4) == E_ARG
    assert _lin_fwd(lib, eta_rule=3, out=None) == E_NULL  # TTT_ETA_DENSE_F32 is a valid rule
    assert _lin_fwd(lib, eta_rule=-1) == E_ARG
    # a valid eta rule passes on to the next check (here: a missing output)
    assert _lin_fwd(lib, eta_rule=LAYER, out=None) == E_NULL
    assert _lin_fwd(lib, eta_rule=CAUSAL, out=None) == E_NULL
    assert _lin_fwd(lib, Wl=P, XQ=None) == E_NULL
    assert _lin_fwd(lib, Wl=P, bl=None, Wc=Q, bc=P, XQ=P, K=16) in (E_NULL, E_ALIGN)


def test_linear_saved_buffer(lib):
    B, H, NC, K, F = 2, 4, 16, 16, 64
    need = lib.ttt_linear_saved_bytes(B, H, NC, K, F)
    # per mini-batch: G, normalised Z1 and Zb (fp32, K x F each) and 3 x 16 statistics padded to 256 bytes
    assert need == B * H * NC * (3 * K * F * 4 + 256)
    assert lib.ttt_linear_saved_bytes(B, H, NC, K, 32) == B * H * NC * (3 * K * 32 * 4 + 256)
    assert lib.ttt_linear_saved_bytes(0, H, NC, K, F) == 0
    assert lib.ttt_linear_saved_bytes(B, H, NC, 8, F) == 0
    # general shapes: the state entering every mini-batch plus fp32 scratch
    gen = lib.ttt_linear_saved_bytes(B, H, NC, 64, 32)
    assert gen >= B * H * NC * (32 * 32 + 32) * 4
    assert _lin_fwd(lib, K=64, F=32, saved=P, saved_bytes=gen - 4) == E_WS
    assert _lin_fwd(lib, saved=P, saved_bytes=need - 4) == E_WS
    assert _lin_fwd(lib, saved=Q, saved_bytes=need) == E_ALIGN
    args = [P] * 9 + [B, H, NC, K, F, 4, F32, DENSE, 1e-8] + [P] * 8
    assert lib.ttt_linear_bwd(*args, P, need - 4, None) == E_WS
    bad = list(args)
    bad[16] = 5  # eta_rule
    assert lib.ttt_linear_bwd(*bad, P, need, None) == E_ARG
    assert lib.ttt_linear_bwd(*args, None, need, None) == E_WS
    assert lib.ttt_linear_bwd(*args, Q, need, None) == E_ALIGN
    bad = list(args)
    bad[8] = None  # dout
    assert lib.ttt_linear_bwd(*bad, P, need, None) == E_NULL
    bad = list(args)
    bad[7] = None  # W1_last
    assert lib.ttt_linear_bwd(*bad, P, need, None) == E_NULL


def _mlp_fwd(lib, FF=256, M=0, memo=(None,) * 4, saved=None, saved_bytes=0, NC=16, ckpt=(None,) * 4, **kw):
    a = ([P] * 10 + [2, 4, NC, 16, 64, FF, 4, M, kw.get("dtype", BF16), kw.get("eta_rule", DENSE), 1e-8, P]
         + [None] * 4 + list(ckpt) + list(memo) + [saved, saved_bytes, None])
    return lib.ttt_mlp_fwd(*a)


def test_mlp_fwd_validation(lib):
    assert _mlp_fwd(lib, FF=72) == E_SHAPE
    assert _mlp_fwd(lib, FF=2048) == E_SHAPE
    # FF = 96 or 512, outside the specialised set, take the general-shape
    # kernels: their forward needs the saved buffer
    assert _mlp_fwd(lib, FF=96) == E_WS
    assert _mlp_fwd(lib, FF=512) == E_WS
    assert _mlp_fwd(lib, dtype=3) == E_DTYPE
    assert _mlp_fwd(lib, memo=(P, P, P, None), M=2) == E_NULL
    assert _mlp_fwd(lib, memo=(P, P, P, P), M=0) == E_ARG
    assert _mlp_fwd(lib, eta_rule=7) == E_ARG
    # M > NC is accepted (one memo state, as the reference's loop gives): the
    # call gets past the memo check to the saved-buffer check
    need = lib.ttt_mlp_saved_bytes(2, 4, 16, 16, 64, 256, BF16)
    assert _mlp_fwd(lib, memo=(P, P, P, P), M=17, saved=Q, saved_bytes=need) == E_ALIGN
    assert _mlp_fwd(lib, memo=(P, P, Q, P), M=2) == E_ALIGN
    # checkpoints: W1's, optionally with any of the other three
    assert _mlp_fwd(lib, ckpt=(None, P, None, None)) == E_NULL
    assert _mlp_fwd(lib, ckpt=(None, None, P, P)) == E_NULL
    assert _mlp_fwd(lib, ckpt=(Q, None, None, None)) == E_ALIGN
    need = lib.ttt_mlp_saved_bytes(2, 4, 16, 16, 64, 256, BF16)
    assert _mlp_fwd(lib, saved=P, saved_bytes=need - 1) == E_WS
    assert _mlp_fwd(lib, saved=Q, saved_bytes=need) == E_ALIGN
    # per-chain slabs must stay addressable with 31-bit byte offsets
    assert _mlp_fwd(lib, NC=40000) == E_SHAPE


def test_mlp_saved_buffer(lib):
    B, H, NC, K, F, FF, G = 2, 4, 16, 16, 64, 256, 8
    n16 = lib.ttt_mlp_saved_bytes(B, H, NC, K, F, FF, BF16)
    n32 = lib.ttt_mlp_saved_bytes(B, H, NC, K, F, FF, F32)
    # per mini-batch: the update operands -e*G1 [K x FF] and -e*G2 [K x F] and
    # six [K x FF] activations (gelu(Z1), gelu'(Z1), G1, Pm gelu''(Z1), gelu(Z1b),
    # gelu'(Z1b)) in the activation type; the fp32 bias decrements, G2 and the
    # two normalised [K x F] rows; four 1 KB fp32 blocks (row statistics, X2b X2^T)
    for n, st in ((n16, 2), (n32, 4)):
        assert n == B * H * NC * ((7 * FF + F) * K * st + (FF + F) * 4 + 3 * K * F * 4 + 4 * 1024)
    assert lib.ttt_mlp_saved_bytes(B, H, NC, K, F, FF, 9) == 0
    assert lib.ttt_mlp_saved_bytes(0, H, NC, K, F, FF, BF16) == 0
    w16 = lib.ttt_mlp_bwd_workspace_bytes(B, H, NC, K, F, FF, BF16)
    # per mini-batch: dZ1b and dZ1 [K x FF] in the activation type, two fp32 [K x F] partials;
    # then the dXQ/dXK workers' control words (4 + one flag per chain and mini-batch, in
    # 256-byte units)
    ctrl = ((4 + B * H * NC) * 4 + 255) // 256 * 256
    assert w16 == B * H * NC * (2 * FF * K * 2 + 2 * K * F * 4) + ctrl
    args = [P] * 15 + [B, H, NC, K, F, FF, G, BF16, DENSE, 1e-8] + [P] * 10
    assert lib.ttt_mlp_bwd(*args, P, n16 - 1, P, w16, None) == E_WS
    bad = list(args)
    bad[23] = 4  # eta_rule
    assert lib.ttt_mlp_bwd(*bad, P, n16, P, w16, None) == E_ARG
    assert lib.ttt_mlp_bwd(*args, None, n16, P, w16, None) == E_WS
    assert lib.ttt_mlp_bwd(*args, Q, n16, P, w16, None) == E_ALIGN
    assert lib.ttt_mlp_bwd(*args, P, n16, P, w16 - 1, None) == E_WS
    assert lib.ttt_mlp_bwd(*args, P, n16, None, w16, None) == E_WS
    bad = list(args)
    bad[10] = None  # W1_last
    assert lib.ttt_mlp_bwd(*bad, P, n16, P, w16, None) == E_NULL


def _readout(lib, **kw):
    a = dict(XQ=P, W1=P, b1=P, W2=P, b2=P, lw=P, lb=P, B=2, H=4, NS=3, K=16, F=64, FF=256, S=1, dtype=BF16,
             eps=1e-6, out=P, stream=None)
    a.update(kw)
    return lib.ttt_mlp_cached_readout(*a.values())


def test_readout_validation(lib):
    assert _readout(lib, K=8) == E_SHAPE
    assert _readout(lib, FF=48) == E_SHAPE
    assert _readout(lib, F=48) == E_SHAPE
    assert _readout(lib, NS=0) == E_SHAPE
    assert _readout(lib, S=0) == E_ARG
    assert _readout(lib, eps=-1.0) == E_ARG
    assert _readout(lib, dtype=3) == E_DTYPE
    assert _readout(lib, W2=None) == E_NULL
    assert _readout(lib, out=Q) == E_ALIGN


def test_fp16_sizes_match_bf16(lib):
    """fp16 activations (TTT_DTYPE_F16) take the bf16 layouts: every
    size helper returns the same byte count for both 16-bit types."""
    for K, F, FF in ((16, 64, 256), (64, 32, 32), (32, 128, 256)):
        assert lib.ttt_mlp_saved_bytes(2, 4, 8, K, F, FF, F16) == lib.ttt_mlp_saved_bytes(2, 4, 8, K, F, FF, BF16) > 0
    assert lib.ttt_mlp_bwd_workspace_bytes(2, 4, 8, 16, 64, 256, F16) == \
        lib.ttt_mlp_bwd_workspace_bytes(2, 4, 8, 16, 64, 256, BF16) > 0
    assert lib.ttt_mlp_memo_workspace_bytes(2, 4, 8, 16, 64, 256, 2, F16) == \
        lib.ttt_mlp_memo_workspace_bytes(2, 4, 8, 16, 64, 256, 2, BF16) > \
        lib.ttt_mlp_memo_workspace_bytes(2, 4, 8, 16, 64, 256, 2, F32)
    assert lib.ttt_mlp_saved_bytes(2, 4, 8, 16, 64, 256, 3) == 0


def test_product_fails_loudly_without_a_gpu():
    """On a host without a GPU the launchers refuse instead of computing on the CPU."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from oracle import ttt_oracle as O
    from ttt_amd.linear import linear_forward
    from ttt_amd.mlp import mlp_cached_readout
    d = O.make_inputs(1, 1, 2, 16, 64, seed=0)
    with pytest.raises(ValueError, match="GPU"):
        linear_forward(d["ln_w"], d["ln_b"], d["W1"], d["b1"], d["XQ"], d["XV"], d["XK"], d["eta"], 1)
    with pytest.raises(ValueError, match="GPU"):
        W = torch.zeros(1, 1, 64, 64)
        mlp_cached_readout(d["XQ"], W, torch.zeros(1, 1, 1, 64), W, torch.zeros(1, 1, 1, 64), d["ln_w"], d["ln_b"])


def test_memo_combine_validation(lib):
    B, H, NC, K, F, FF, M = 2, 3, 10, 16, 64, 256, 3
    NS = -(-NC // M)
    need = lib.ttt_mlp_memo_gates_bytes(B, H, NC, K, F, M)
    per_chain = 2 * NS * NC * K + 2 * NC * K + NS * F
    assert need == B * H * ((per_chain + 3) // 4 * 4) * 4
    assert lib.ttt_mlp_memo_gates_bytes(B, H, NC, K, F, 0) == 0
    assert lib.ttt_mlp_memo_gates_bytes(B, H, NC, K, 48, M) == 0
    # the full workspace: bf16 adds one LDS image per memo state (W1, W2 as bf16
    # operand frags, fp32 biases, padded to whole kilobytes) behind the gates
    img = -(-(2 * F * FF * 2 + (FF + F) * 4) // 1024) * 1024
    assert lib.ttt_mlp_memo_workspace_bytes(B, H, NC, K, F, FF, M, BF16) == -(-need // 256) * 256 + B * H * NS * img
    assert lib.ttt_mlp_memo_workspace_bytes(B, H, NC, K, F, FF, M, F32) == need
    assert lib.ttt_mlp_memo_workspace_bytes(B, H, NC, K, F, 96, M, BF16) == 0

    def fwd(**kw):
        a = dict(ptrs=[P] * 10, B=B, H=H, NC=NC, K=K, F=F, FF=FF, M=M, dtype=BF16, eps=1e-6, out=P, gates=P,
                 gb=need, stream=None)
        a.update(kw)
        return lib.ttt_mlp_memo_combine(*a["ptrs"], a["B"], a["H"], a["NC"], a["K"], a["F"], a["FF"], a["M"],
                                        a["dtype"], a["eps"], a["out"], a["gates"], a["gb"], a["stream"])
    assert fwd(FF=96) == E_SHAPE
    assert fwd(M=0) == E_ARG
    assert fwd(NC=300, M=1) == E_SHAPE  # more than 256 memo states
    assert fwd(gb=need - 4) == E_WS
    assert fwd(gates=None) == E_WS
    assert fwd(gates=Q) == E_ALIGN
    assert fwd(out=None) == E_NULL
    assert fwd(ptrs=[P] * 2 + [None] + [P] * 7) == E_NULL
    assert fwd(dtype=5) == E_DTYPE
    bwd = [P] * 10 + [B, H, NC, K, F, FF, M, BF16, 1e-6]
    assert lib.ttt_mlp_memo_combine_bwd(*bwd, P, need - 4, P, P, P, None) == E_WS
    assert lib.ttt_mlp_memo_combine_bwd(*bwd, P, need, None, P, P, None) == E_NULL
    assert lib.ttt_mlp_memo_combine_bwd(*bwd, P, need, P, None, P, None) == E_NULL
    assert lib.ttt_mlp_memo_combine_bwd(*([P, None] + [P] * 8 + bwd[10:]), P, need, P, P, P, None) == E_NULL


def test_options(lib):
    from ttt_amd import _lib
    poll, fused = _lib.OPT_MLP_BWD_POLL_LIMIT, _lib.OPT_MLP_BWD_FUSED
    old_poll, old_fused = lib.ttt_get_option(poll), lib.ttt_get_option(fused)
    assert old_poll == 1 << 22 and old_fused == 1
    try:
        assert lib.ttt_set_option(poll, 0) == OK and lib.ttt_get_option(poll) == 0
        assert lib.ttt_set_option(poll, -1) == E_ARG
        assert lib.ttt_set_option(poll, 1 << 31) == E_ARG
        assert lib.ttt_set_option(fused, 0) == OK and lib.ttt_get_option(fused) == 0
        assert lib.ttt_set_option(fused, 2) == E_ARG
        assert lib.ttt_set_option(99, 1) == E_ARG
        assert lib.ttt_get_option(99) == -1
        small = _lib.OPT_SMALL_KERNELS
        assert lib.ttt_get_option(small) == 1
        assert lib.ttt_set_option(small, 0) == OK and lib.ttt_get_option(small) == 0
        assert lib.ttt_set_option(small, 3) == E_ARG
    finally:
        lib.ttt_set_option(poll, old_poll)
        lib.ttt_set_option(fused, old_fused)
        lib.ttt_set_option(_lib.OPT_SMALL_KERNELS, 1)


def test_mlp_bwd_check_validation(lib):
    B, H, NC, K, F, FF = 2, 4, 16, 16, 64, 256
    w = lib.ttt_mlp_bwd_workspace_bytes(B, H, NC, K, F, FF, BF16)
    # NULL names the no-allocation entry point's scratch: a problem larger than it is refused on the host
    assert lib.ttt_mlp_bwd_check(None, 0, 16, 12, 128, K, F, FF, BF16, None) == -9
    assert lib.ttt_mlp_bwd_check(P, w - 1, B, H, NC, K, F, FF, BF16, None) == E_WS
    assert lib.ttt_mlp_bwd_check(P, w, 0, H, NC, K, F, FF, BF16, None) == E_SHAPE


def test_model_config_rejects_shapes_the_layer_kernels_do_not_take():
    """ModelConfig raises before any layer is built: head dims other than 32
    and 64 (producer, post-norm, memory cache), model widths above 1024, and
    mini-batches that are not 16..64 tokens in steps of 16."""
    from ttt_amd.model import ModelConfig
    ModelConfig(seq_len=512, model_dim=128, num_heads=4, mini_batch_size=64)   # main.py's shape
    ModelConfig(seq_len=512, model_dim=1024, num_heads=16, mini_batch_size=16)
    for kw in (dict(model_dim=192, num_heads=4),      # F = 48
               dict(model_dim=128, num_heads=1),      # F = 128
               dict(model_dim=2048, num_heads=32),    # F = 64, D > 1024
               dict(model_dim=128, num_heads=4, mini_batch_size=8, seq_len=512),
               dict(model_dim=128, num_heads=4, mini_batch_size=128, seq_len=512)):
        with pytest.raises(ValueError):
            ModelConfig(**{"seq_len": 512, "mini_batch_size": 64, **kw})
