"""GPU parity of the Qwen3.5 layer primitives (row norms, convolution step,
recurrent parameters, IMROPE, SiLU) and of the two fused decode-step entry
points (attention prologue, recurrent-layer step) against the fp64 oracle
(oracle/layer.py).  Tolerances: fp32 results 1e-4, fp16/bf16 results 2e-2;
pure copies (cache values, convolution history) bit-exact."""

import importlib

import numpy as np
import pytest

from oracle import attention as A
from oracle import inputs as I
from oracle import layer as L

pytestmark = pytest.mark.gpu


def _mod(name):
    return importlib.import_module("alpacca-open-sourced-by-jt_amd." + name)


def _td(torch, name):
    return {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[name]


def _dev(torch, arr, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32)).to(device).to(
        _td(torch, dtype))


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _tol(dtype):
    return 1e-4 if dtype == "f32" else 2e-2


@pytest.fixture(scope="module")
def ops(gpu):
    return _mod("qwen35_rocm_ops").Qwen35RocmOps()


# ------------------------------------------------------------ row norms

@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n", [128, 256, 100, 1, 700])
def test_rms_l2_gated_norms(gpu, ops, dtype, n):
    import torch
    rng = np.random.default_rng(n)
    x = I.round_to(rng.standard_normal((3, 5, n)) * 2.0, dtype)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    gt = I.round_to(rng.standard_normal((3, 5, n)), dtype)
    X, G_ = _dev(torch, x, dtype, gpu), _dev(torch, gt, dtype, gpu)
    W = torch.from_numpy(w).to(gpu)
    got = ops.rms_norm(X, W, 1e-6)
    assert got.dtype == X.dtype and tuple(got.shape) == x.shape
    assert np.abs(_np(got) - L.rms_norm(x, w, 1e-6)).max() <= _tol(dtype)
    got = ops.l2_normalize(X, 1e-6)
    assert np.abs(_np(got) - L.l2_normalize(x, 1e-6)).max() <= _tol(dtype)
    got = ops.recurrent_gate(X, W, G_, 1e-6)
    assert np.abs(_np(got) - L.gated_rms_norm(x, w, gt, 1e-6)).max() <= _tol(dtype)


def test_l2_norm_of_zero_rows_and_tiny_rows(gpu, ops):
    import torch
    x = np.zeros((4, 64), dtype=np.float32)
    x[1, 3] = 1e-8
    x[2] = 1.0
    got = ops.l2_normalize(torch.from_numpy(x).to(gpu), 1e-6).cpu().numpy()
    np.testing.assert_allclose(got, L.l2_normalize(x, 1e-6), atol=1e-6)
    assert got[0].max() == 0.0


def test_grouped_row_addressing(gpu):
    # q and k heads read straight out of the convolution output [B, C]
    import torch
    ops_mod = _mod("_ops")
    lib = _mod("_lib")
    rng = np.random.default_rng(3)
    b, hk, dk, rest = 3, 4, 32, 50
    c = 2 * hk * dk + rest
    x = rng.standard_normal((b, c)).astype(np.float32)
    X = torch.from_numpy(x).to(gpu)
    out = ops_mod.row_norm(X, mode=lib.NORM_L2, eps=1e-6, n=dk, rows=b * hk, group_rows=hk,
                           group_stride=c)
    ref = L.l2_normalize(x[:, :hk * dk].reshape(b * hk, dk), 1e-6)
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-5
    assert np.array_equal(X.cpu().numpy(), x)  # the input is only read


def test_silu(gpu, ops):
    import torch
    x = np.linspace(-90, 90, 1001).astype(np.float32)
    got = ops.silu(torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert np.abs(got - L.silu(x)).max() <= 1e-4


# ------------------------------------------------------------ conv step

@pytest.mark.parametrize("kernel", [4, 2, 1])
def test_causal_convolution_step_rocm(gpu, ops, kernel):
    import torch
    rng = np.random.default_rng(kernel)
    b, c = 3, 8192 + 5
    cur = rng.standard_normal((b, c)).astype(np.float32)
    w = rng.standard_normal((kernel, c)).astype(np.float32)
    hist = rng.standard_normal((b, kernel - 1, c)).astype(np.float32)
    H = torch.from_numpy(hist).to(gpu)
    out = ops.causal_convolution_step_(torch.from_numpy(cur).to(gpu), torch.from_numpy(w).to(gpu), H)
    ref, new_hist = L.conv_step(cur, w, hist)
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-4
    assert np.array_equal(H.cpu().numpy(), new_hist.astype(np.float32))  # shift is a copy


def test_qwen35_conv_step_numpy_in_place(gpu):
    K = _mod("qwen35_kernels")
    rng = np.random.default_rng(9)
    c, kernel = 300, 4
    cur = rng.standard_normal(c).astype(np.float32)
    w = rng.standard_normal((c, kernel)).astype(np.float32)  # [C, K] order of qwen35_kernels
    hist = rng.standard_normal((kernel - 1, c)).astype(np.float32)
    h0 = hist.copy()
    out, hist_ret = K.qwen35_conv_step(cur, w, hist)
    ref, new_hist = L.conv_step(cur, w, h0, layout="ck", apply_silu=True)
    assert hist_ret is hist
    assert np.abs(out - ref).max() <= 1e-4
    assert np.array_equal(hist, new_hist.astype(np.float32))


# --------------------------------------------------- recurrent parameters

def test_recurrent_parameters(gpu, ops):
    import torch
    rng = np.random.default_rng(11)
    b, h = 5, 32
    bl = (rng.standard_normal((b, h)) * 8).astype(np.float32)
    al = (rng.standard_normal((b, h)) * 8).astype(np.float32)
    dt = rng.standard_normal(h).astype(np.float32)
    ssm = (-np.exp(rng.uniform(-1, 1, h))).astype(np.float32)
    beta, g = ops.recurrent_parameters(*(torch.from_numpy(x).to(gpu) for x in (bl, al, dt, ssm)))
    rb, rg = L.recurrent_parameters(bl, al, dt, ssm)
    assert np.abs(beta.cpu().numpy() - rb).max() <= 1e-5
    assert np.abs(g.cpu().numpy() - rg).max() <= 1e-4 * max(1.0, np.abs(rg).max())


def test_qwen35_normalize_qk_and_beta_decay_numpy(gpu):
    K = _mod("qwen35_kernels")
    rng = np.random.default_rng(12)
    q = rng.standard_normal((16, 128)).astype(np.float32)
    k = rng.standard_normal((16, 128)).astype(np.float32)
    qn, kn = K.qwen35_normalize_qk(q, k, 1e-6)
    assert np.abs(qn - L.l2_normalize(q, 1e-6)).max() <= 1e-5
    assert np.abs(kn - L.l2_normalize(k, 1e-6)).max() <= 1e-5
    args = [rng.standard_normal(32).astype(np.float32) for _ in range(3)]
    ssm = (-np.exp(rng.uniform(-1, 1, 32))).astype(np.float32)
    beta, g = K.qwen35_beta_decay(*args, ssm)
    rb, rg = L.recurrent_parameters(args[0], args[1], args[2], ssm)
    assert np.abs(beta - rb).max() <= 1e-5 and np.abs(g - rg).max() <= 1e-4


# ----------------------------------------------------------------- IMROPE

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_imrope_rocm_single_lane_vector(gpu, ops, dtype):
    import torch
    rng = np.random.default_rng(13)
    x = I.round_to(rng.standard_normal((4, 16, 256)), dtype)
    lanes = np.array([32767, 32767, 32767, 0], dtype=np.int64)
    got = ops.imrope(_dev(torch, x, dtype, gpu), torch.from_numpy(lanes).to(gpu),
                     (11, 11, 10, 0), frequency_base=10000000.0)
    ref = L.imrope(x, lanes.astype(np.float64), (11, 11, 10, 0), 10000000.0)
    assert np.abs(_np(got) - ref).max() <= _tol(dtype)
    if dtype == "f32":  # coordinates past 2 R are copied bit-exactly
        assert np.array_equal(got[..., 64:].cpu().numpy(), x[..., 64:])


def test_imrope_per_row_lanes_and_scale(gpu, ops):
    import torch
    rng = np.random.default_rng(14)
    rows, d = 37, 24
    x = rng.standard_normal((rows, d)).astype(np.float32)
    lanes = rng.integers(0, 100000, (rows, 4)).astype(np.int64)
    got = ops.imrope(torch.from_numpy(x).to(gpu), torch.from_numpy(lanes).to(gpu), (2, 3, 1, 4),
                     frequency_base=500000.0, frequency_scale=0.25)
    ref = L.imrope(x, lanes.astype(np.float64), (2, 3, 1, 4), 500000.0, scale=0.25)
    assert np.abs(got.cpu().numpy() - ref).max() <= 1e-4


# ------------------------------------------------- attention prologue

@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_attention_prologue_then_gated_decode(gpu, ops, dtype):
    # Qwen3.5 full-attention decode step on the C4 head geometry: prologue
    # (split + Q/K RMSNorm + IMROPE + append) then split-K decode with the
    # fused sigmoid gate, against the oracle on the same rounded inputs
    import torch
    rng = np.random.default_rng(15)
    b, hq, hkv, d, cap, pos = 4, 16, 2, 256, 640, 600
    sections, base, eps = (11, 11, 10, 0), 10000000.0, 1e-6
    kc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    vc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    qg = I.round_to(rng.standard_normal((b, hq * 2 * d)) * 3, dtype)
    k = I.round_to(rng.standard_normal((b, hkv * d)) * 3, dtype)
    v = I.round_to(rng.standard_normal((b, hkv * d)), dtype)
    qw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    KC, VC = _dev(torch, kc, dtype, gpu), _dev(torch, vc, dtype, gpu)
    q_dev, gate_dev, nxt = ops.attention_prologue_(
        _dev(torch, qg, dtype, gpu), _dev(torch, k, dtype, gpu), _dev(torch, v, dtype, gpu),
        torch.from_numpy(qw).to(gpu), torch.from_numpy(kw).to(gpu), KC, VC, position=pos,
        sections=sections, frequency_base=base, epsilon=eps)
    assert nxt == pos + 1
    rq, rg, rk, rv = L.attention_prologue(qg, k, v, qw, kw, eps, np.full(b, pos), sections, base)
    tol = _tol(dtype)
    assert np.abs(_np(q_dev) - rq).max() <= tol
    assert np.array_equal(_np(gate_dev), rg)
    got_k = _np(KC)
    assert np.abs(got_k[pos] - rk).max() <= tol
    assert np.array_equal(_np(VC)[pos], rv)
    # untouched rows stay bit-identical
    assert np.array_equal(np.delete(got_k, pos, axis=0), np.delete(kc, pos, axis=0))
    out = ops.online_attention(q_dev, KC, VC, length=pos + 1, gate=gate_dev)
    # oracle decode on what the device wrote (the cache row is the device's
    # rounded key; the query is the device's rounded query)
    kc_dev, vc_dev, q_used = got_k, _np(VC), _np(q_dev)
    for bb in range(b):
        ref = A.attention_decode_twopass(q_used[bb], kc_dev[:pos + 1, bb], vc_dev[:pos + 1, bb],
                                         hq // hkv, 1.0 / 16.0)
        ref = ref * (1.0 / (1.0 + np.exp(-rg[bb])))
        assert np.abs(_np(out[bb]) - ref).max() <= tol


# (b, hq, hkv, d, cap, pos): the Qwen3.5 C4 geometry; head_dim 128 at group
# 8; group 40 at head_dim 64 (three 16-head column blocks, so three blocks
# hold the new row and only the first writes it); position 0 (one cache
# row); a position on a split-chunk edge.
_STEP_SHAPES = [(4, 16, 2, 256, 640, 600), (2, 16, 2, 128, 300, 257),
                (1, 40, 1, 64, 200, 130), (3, 8, 2, 128, 64, 0), (1, 16, 2, 256, 4096, 3071)]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("b,hq,hkv,d,cap,pos", _STEP_SHAPES)
def test_attention_layer_step_fused_equals_two_calls(gpu, ops, dtype, b, hq, hkv, d, cap, pos):
    """The fused step (prologue inside the split-K launch, gate read from
    the joint projection in the combine) returns the bytes of
    attention_prologue_ + online_attention(gate=) and leaves the caches in
    the same state; both match the oracle."""
    import torch
    rng = np.random.default_rng(b * 1000 + hq * 10 + d + pos)
    sections, base, eps = (11, 11, 10, 0), 10000000.0, 1e-6
    if 2 * sum(sections) > d:
        sections = (4, 4, 2, 0)
    kc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    vc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    qg = I.round_to(rng.standard_normal((b, hq * 2 * d)) * 3, dtype)
    k = I.round_to(rng.standard_normal((b, hkv * d)) * 3, dtype)
    v = I.round_to(rng.standard_normal((b, hkv * d)), dtype)
    qw = torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(gpu)
    kw = torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(gpu)
    args = (_dev(torch, qg, dtype, gpu), _dev(torch, k, dtype, gpu), _dev(torch, v, dtype, gpu),
            qw, kw)
    kw_args = dict(position=pos, sections=sections, frequency_base=base, epsilon=eps)
    KC1, VC1 = _dev(torch, kc, dtype, gpu), _dev(torch, vc, dtype, gpu)
    q_dev, gate_dev, nxt = ops.attention_prologue_(*args, KC1, VC1, **kw_args)
    two = ops.online_attention(q_dev, KC1, VC1, length=nxt, gate=gate_dev)
    two32 = ops.online_attention(q_dev, KC1, VC1, length=nxt, gate=gate_dev,
                                 out_dtype=torch.float32)
    KC2, VC2 = _dev(torch, kc, dtype, gpu), _dev(torch, vc, dtype, gpu)
    fused, n2 = ops.attention_layer_step_(*args, KC2, VC2, **kw_args)
    fused32, _ = ops.attention_layer_step_(*args, KC2, VC2, out_dtype=torch.float32, **kw_args)
    torch.cuda.synchronize()
    assert n2 == nxt == pos + 1
    assert fused.dtype == _td(torch, dtype) and fused.shape == (b, hq, d)
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))
    assert torch.equal(fused32, two32)
    assert torch.equal(KC2.view(torch.int16), KC1.view(torch.int16))
    assert torch.equal(VC2.view(torch.int16), VC1.view(torch.int16))
    # against the oracle: prologue on the host inputs, decode on the cache
    # the device wrote
    rq, rg, rk, rv = L.attention_prologue(qg, k, v, _np(qw), _np(kw), eps, np.full(b, pos),
                                          sections, base)
    tol = _tol(dtype)
    got_k = _np(KC2)
    assert np.abs(got_k[pos] - rk).max() <= tol
    assert np.array_equal(_np(VC2)[pos], rv)
    vc_dev = _np(VC2)
    for bb in range(b):
        ref = A.attention_decode_twopass(rq[bb], got_k[:pos + 1, bb], vc_dev[:pos + 1, bb],
                                         hq // hkv, 1.0 / np.sqrt(d))
        ref = ref * (1.0 / (1.0 + np.exp(-rg[bb])))
        assert np.abs(_np(fused32[bb]) - ref).max() <= tol


@pytest.mark.parametrize("dtype,d,rows,bound", [("bf16", 256, (600, 17, 0, 333), 600),
                                                ("f16", 128, (5, 290, 64), 299),
                                                ("f32", 64, (40, 3), 70)])
def test_attention_layer_step_ragged_positions(gpu, ops, dtype, d, rows, bound):
    """Per-sequence rows (a ragged batch): the fused step equals the
    prologue with positions + the gated decode with seq_lens = row + 1 bit
    for bit (fp32 takes those two calls itself), and both match the
    oracle per sequence."""
    import torch
    rng = np.random.default_rng(d + len(rows))
    b, hq, hkv, cap = len(rows), 16, 2, bound + 40
    sections, base, eps = (11, 11, 10, 0), 10000000.0, 1e-6
    if 2 * sum(sections) > d:
        sections = (4, 4, 2, 0)
    kc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    vc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    qg = I.round_to(rng.standard_normal((b, hq * 2 * d)) * 3, dtype)
    k = I.round_to(rng.standard_normal((b, hkv * d)) * 3, dtype)
    v = I.round_to(rng.standard_normal((b, hkv * d)), dtype)
    qw_h = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kw_h = rng.uniform(0.5, 1.5, d).astype(np.float32)
    qw, kw = torch.from_numpy(qw_h).to(gpu), torch.from_numpy(kw_h).to(gpu)
    args = (_dev(torch, qg, dtype, gpu), _dev(torch, k, dtype, gpu), _dev(torch, v, dtype, gpu),
            qw, kw)
    pos_dev = torch.tensor(rows, dtype=torch.int32, device=gpu)
    KC2, VC2 = _dev(torch, kc, dtype, gpu), _dev(torch, vc, dtype, gpu)
    fused, n = ops.attention_layer_step_(*args, KC2, VC2, position=bound, positions=list(rows),
                                         sections=sections, frequency_base=base, epsilon=eps,
                                         out_dtype=torch.float32)
    assert n == bound + 1
    if dtype != "f32":
        KC1, VC1 = _dev(torch, kc, dtype, gpu), _dev(torch, vc, dtype, gpu)
        q_dev, gate_dev = _mod("_ops").attention_prologue(
            args[0].reshape(b, hq, 2 * d), args[1], args[2], qw, kw, KC1, VC1, position=bound,
            positions=pos_dev, sections=sections, frequency_base=base, eps=eps)
        two = ops.online_attention(q_dev, KC1, VC1, length=bound + 1, seq_lens=pos_dev + 1,
                                   gate=gate_dev, out_dtype=torch.float32)
        fused_dev, _ = ops.attention_layer_step_(*args, _dev(torch, kc, dtype, gpu),
                                                 _dev(torch, vc, dtype, gpu), position=bound,
                                                 positions=pos_dev, sections=sections,
                                                 frequency_base=base, epsilon=eps,
                                                 out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(fused, two) and torch.equal(fused_dev, two)
        assert torch.equal(KC2.view(torch.int16), KC1.view(torch.int16))
        assert torch.equal(VC2.view(torch.int16), VC1.view(torch.int16))
    rq, rg, rk, rv = L.attention_prologue(qg, k, v, qw_h, kw_h, eps, np.array(rows), sections,
                                          base)
    tol = _tol(dtype)
    got_k, got_v = _np(KC2), _np(VC2)
    for bb, p in enumerate(rows):
        assert np.abs(got_k[p, bb] - rk[bb]).max() <= tol
        assert np.array_equal(got_v[p, bb], rv[bb])
        ref = A.attention_decode_twopass(rq[bb], got_k[:p + 1, bb], got_v[:p + 1, bb],
                                         hq // hkv, 1.0 / np.sqrt(d))
        ref = ref * (1.0 / (1.0 + np.exp(-rg[bb])))
        assert np.abs(_np(fused[bb]) - ref).max() <= tol
    # the rows other sequences' tokens went to are untouched
    mask = np.ones((cap, b), bool)
    mask[list(rows), np.arange(b)] = False
    assert np.array_equal(got_k[mask], kc[mask])


@pytest.mark.parametrize("dtype,d", [("bf16", 128), ("f32", 128), ("f32", 96)])
def test_attention_layer_step_device_position_past_the_step(gpu, ops, dtype, d):
    """A device position beyond the step's `position` (but inside the
    cache) writes no cache row on either form of the step -- the fused
    kernel (fp16 / bf16, widths 64 / 128 / 256) and the prologue + gated
    decode pair (fp32 and other widths) -- and that sequence attends to the
    step's position + 1 rows, as the device lengths are clamped there."""
    import torch
    rng = np.random.default_rng(500 + d + len(dtype))
    b, hq, hkv, cap, position = 3, 8, 2, 96, 40
    rows = [12, 70, 40]  # sequence 1's device row lies past `position`
    sections, base, eps = (4, 4, 2, 0), 10000.0, 1e-6
    kc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    vc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dtype)
    qg = I.round_to(rng.standard_normal((b, hq * 2 * d)) * 3, dtype)
    k = I.round_to(rng.standard_normal((b, hkv * d)) * 3, dtype)
    v = I.round_to(rng.standard_normal((b, hkv * d)), dtype)
    qw_h = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kw_h = rng.uniform(0.5, 1.5, d).astype(np.float32)
    KC, VC = _dev(torch, kc, dtype, gpu), _dev(torch, vc, dtype, gpu)
    out, n = ops.attention_layer_step_(
        _dev(torch, qg, dtype, gpu), _dev(torch, k, dtype, gpu), _dev(torch, v, dtype, gpu),
        torch.from_numpy(qw_h).to(gpu), torch.from_numpy(kw_h).to(gpu), KC, VC,
        position=position, positions=torch.tensor(rows, dtype=torch.int32, device=gpu),
        sections=sections, frequency_base=base, epsilon=eps, out_dtype=torch.float32)
    assert n == position + 1
    got_k, got_v = _np(KC), _np(VC)
    # sequence 1 wrote nothing; every row but the two written ones is untouched
    mask = np.ones((cap, b), bool)
    mask[[12, 40], [0, 2]] = False
    assert np.array_equal(got_k[mask], kc[mask])
    assert np.array_equal(got_v[mask], vc[mask])
    rq, rg, rk, rv = L.attention_prologue(qg, k, v, qw_h, kw_h, eps, np.array(rows), sections,
                                          base)
    tol = _tol(dtype)
    for bb, p in enumerate(rows):
        n_rows = min(p, position) + 1
        ref = A.attention_decode_twopass(rq[bb], got_k[:n_rows, bb], got_v[:n_rows, bb],
                                         hq // hkv, 1.0 / np.sqrt(d))
        ref = ref * (1.0 / (1.0 + np.exp(-rg[bb])))
        assert np.abs(_np(out[bb]) - ref).max() <= tol, bb


def test_attention_layer_step_rejects_bad_positions(gpu, ops):
    import torch
    b, hq, hkv, d, cap = 2, 8, 2, 128, 64
    z = lambda *shape: torch.zeros(shape, dtype=torch.bfloat16, device=gpu)  # noqa: E731
    w = torch.ones(d, device=gpu)
    args = (z(b, hq * 2 * d), z(b, hkv * d), z(b, hkv * d), w, w, z(cap, b, hkv, d),
            z(cap, b, hkv, d))
    rope = dict(sections=(11, 11, 10, 0), frequency_base=1e7, epsilon=1e-6)
    with pytest.raises(ValueError, match="one row in"):
        ops.attention_layer_step_(*args, position=20, positions=[3, 21], **rope)
    with pytest.raises(ValueError, match="one row in"):
        ops.attention_layer_step_(*args, position=20, positions=[3], **rope)
    with pytest.raises(ValueError, match="one row per sequence"):
        ops.attention_layer_step_(*args, position=20,
                                  positions=torch.zeros(3, dtype=torch.int32, device=gpu), **rope)
    with pytest.raises(ValueError, match="exceeds capacity"):
        ops.attention_layer_step_(*args, position=cap, **rope)


def test_layer_steps_decode_loop_in_a_graph(gpu, ops):
    """A decode loop as one captured graph replayed per token: an attention
    layer step (reading device positions) and a recurrent layer step, whose
    inputs the host refreshes between replays (the attention split plan is
    sized for the whole cache).  Every replay equals the eager steps bit for
    bit, with eager work and synchronisation between replays, and the
    caches and recurrent state end identical."""
    import torch
    g = torch.Generator(device=gpu).manual_seed(21)
    bf = torch.bfloat16
    b, hq, hkv, d, cap = 2, 16, 2, 256, 192
    rope = dict(sections=(11, 11, 10, 0), frequency_base=10000000.0, epsilon=1e-6)
    KG = torch.randn((cap, b, hkv, d), generator=g, device=gpu).to(bf)
    VG = torch.randn((cap, b, hkv, d), generator=g, device=gpu).to(bf)
    qg = torch.zeros((b, hq * 2 * d), dtype=bf, device=gpu)
    kn = torch.zeros((b, hkv * d), dtype=bf, device=gpu)
    vn = torch.zeros((b, hkv * d), dtype=bf, device=gpu)
    qw = torch.rand((d,), generator=g, device=gpu) + 0.5
    kw = torch.rand((d,), generator=g, device=gpu) + 0.5
    pos = torch.tensor([5, 9], dtype=torch.int32, device=gpu)
    hk, hv, dk, dv, kern = 4, 8, 64, 64, 4
    chn = 2 * hk * dk + hv * dv

    def rec_ws():
        return ops.initialize_recurrent_workspace(batch_size=b, convolution_kernel=kern,
                                                  convolution_channels=chn, value_heads=hv,
                                                  value_dimension=dv, key_dimension=dk)

    wg = rec_ws()
    wg.delta_state.copy_(torch.randn(wg.delta_state.shape, generator=g, device=gpu) * 0.1)
    mixed = torch.zeros((b, chn), device=gpu)
    cw = torch.randn((kern, chn), generator=g, device=gpu) * 0.5
    rgate = torch.zeros((b, hv * dv), device=gpu)
    bl = torch.zeros((b, hv), device=gpu)
    al = torch.zeros((b, hv), device=gpu)
    dt = torch.randn((hv,), generator=g, device=gpu)
    ssm = -torch.exp(torch.rand((hv,), generator=g, device=gpu) * 2 - 1)
    nw = torch.rand((dv,), generator=g, device=gpu) + 0.5

    def step(K, V, w):
        out = ops.attention_layer_step_(qg, kn, vn, qw, kw, K, V, position=cap - 1,
                                        positions=pos, **rope)[0]
        rec = ops.recurrent_layer_step_(w, mixed, cw, rgate, bl, al, dt, ssm, nw, key_heads=hk,
                                        key_dimension=dk, epsilon=1e-6)
        return out, rec

    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        for _ in range(2):
            step(KG, VG, wg)
    torch.cuda.current_stream(gpu).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, rec_g = step(KG, VG, wg)
    KE, VE = KG.clone(), VG.clone()
    we = rec_ws()
    we.delta_state.copy_(wg.delta_state)
    we.convolution_history.copy_(wg.convolution_history)
    for i in range(6):
        pos.copy_(torch.tensor([10 + 17 * i, 40 + 3 * i], dtype=torch.int32))
        qg.copy_(torch.randn(qg.shape, generator=g, device=gpu) * 3)
        kn.copy_(torch.randn(kn.shape, generator=g, device=gpu) * 3)
        vn.copy_(torch.randn(vn.shape, generator=g, device=gpu))
        for t in (mixed, rgate, bl, al):
            t.copy_(torch.randn(t.shape, generator=g, device=gpu))
        graph.replay()
        torch.cuda.synchronize()
        out_e, rec_e = step(KE, VE, we)
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16)), i
        assert torch.equal(rec_g, rec_e), i
    assert torch.equal(KG.view(torch.int16), KE.view(torch.int16))
    assert torch.equal(VG.view(torch.int16), VE.view(torch.int16))
    assert torch.equal(wg.delta_state, we.delta_state)
    assert torch.equal(wg.convolution_history, we.convolution_history)


def test_attention_layer_step_fp32_runs_two_calls(gpu, ops):
    """fp32 caches take the separate prologue + gated decode launches."""
    import torch
    rng = np.random.default_rng(3)
    b, hq, hkv, d, cap, pos = 2, 8, 2, 64, 100, 70
    sections, base, eps = (4, 4, 2, 0), 10000.0, 1e-6
    kc = rng.standard_normal((cap, b, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((cap, b, hkv, d)).astype(np.float32)
    qg = rng.standard_normal((b, hq * 2 * d)).astype(np.float32)
    k = rng.standard_normal((b, hkv * d)).astype(np.float32)
    v = rng.standard_normal((b, hkv * d)).astype(np.float32)
    qw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    KC, VC = _dev(torch, kc, "f32", gpu), _dev(torch, vc, "f32", gpu)
    out, n = ops.attention_layer_step_(
        _dev(torch, qg, "f32", gpu), _dev(torch, k, "f32", gpu), _dev(torch, v, "f32", gpu),
        torch.from_numpy(qw).to(gpu), torch.from_numpy(kw).to(gpu), KC, VC, position=pos,
        sections=sections, frequency_base=base, epsilon=eps)
    assert n == pos + 1
    rq, rg, rk, rv = L.attention_prologue(qg, k, v, qw, kw, eps, np.full(b, pos), sections, base)
    got_k, got_v = _np(KC), _np(VC)
    assert np.abs(got_k[pos] - rk).max() <= 1e-4
    for bb in range(b):
        ref = A.attention_decode_twopass(rq[bb], got_k[:pos + 1, bb], got_v[:pos + 1, bb],
                                         hq // hkv, 1.0 / 8.0)
        ref = ref * (1.0 / (1.0 + np.exp(-rg[bb])))
        assert np.abs(_np(out[bb]) - ref).max() <= 1e-4


# ------------------------------------------------ recurrent-layer step

# (1, 1, 2, 64, 300, 3): value rows wider than the one-launch step takes,
# so the prep / GDN step / norm launches run.
@pytest.mark.parametrize("batch,hk,hv,dk,dv,kernel", [(1, 16, 32, 128, 128, 4),
                                                      (2, 2, 4, 64, 96, 4),
                                                      (3, 1, 2, 256, 40, 4), (2, 2, 4, 64, 32, 6),
                                                      (1, 2, 2, 32, 32, 2), (1, 2, 2, 32, 32, 1),
                                                      (1, 1, 2, 64, 300, 3)])
def test_recurrent_layer_step_matches_oracle_over_tokens(gpu, ops, batch, hk, hv, dk, dv, kernel):
    import torch
    rng = np.random.default_rng(batch * 100 + hk + kernel)
    eps, steps = 1e-6, 6
    chn = 2 * hk * dk + hv * dv
    w = (rng.standard_normal((kernel, chn)) * 0.5).astype(np.float32)
    dt = rng.standard_normal(hv).astype(np.float32)
    ssm = (-np.exp(rng.uniform(-1, 1, hv))).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, dv).astype(np.float32)
    ws = ops.initialize_recurrent_workspace(batch_size=batch, convolution_kernel=kernel,
                                            convolution_channels=chn, value_heads=hv,
                                            value_dimension=dv, key_dimension=dk)
    hist = np.zeros((batch, kernel - 1, chn))
    state = np.zeros((batch, hv, dv, dk))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(gpu)  # noqa: E731
    for _ in range(steps):
        mixed = rng.standard_normal((batch, chn)).astype(np.float32)
        gate = rng.standard_normal((batch, hv * dv)).astype(np.float32)
        bl = rng.standard_normal((batch, hv)).astype(np.float32)
        al = rng.standard_normal((batch, hv)).astype(np.float32)
        out = ops.recurrent_layer_step_(ws, T(mixed), T(w), T(gate), T(bl), T(al), T(dt), T(ssm),
                                        T(nw), key_heads=hk, key_dimension=dk, epsilon=eps)
        ref, hist = L.recurrent_layer_step(mixed, w, hist, gate, bl, al, dt, ssm, nw, state,
                                           key_heads=hk, key_dim=dk, value_heads=hv,
                                           value_dim=dv, eps=eps)
        assert np.abs(out.cpu().numpy() - ref).max() <= 1e-4
    assert np.abs(ws.delta_state.cpu().numpy() - state).max() <= 1e-4
    assert np.array_equal(ws.convolution_history.cpu().numpy(), hist.astype(np.float32))


def _recurrent_run(ops, torch, gpu, rng_seed, batch, hk, hv, dk, dv, kernel, out_dtype, steps):
    """Runs `steps` recurrent-layer steps on a fresh workspace; returns the
    outputs and the final state and convolution history (host copies)."""
    rng = np.random.default_rng(rng_seed)
    chn = 2 * hk * dk + hv * dv
    w = (rng.standard_normal((kernel, chn)) * 0.5).astype(np.float32)
    dt = rng.standard_normal(hv).astype(np.float32)
    ssm = (-np.exp(rng.uniform(-1, 1, hv))).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, dv).astype(np.float32)
    ws = ops.initialize_recurrent_workspace(batch_size=batch, convolution_kernel=kernel,
                                            convolution_channels=chn, value_heads=hv,
                                            value_dimension=dv, key_dimension=dk)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(gpu)  # noqa: E731
    outs = []
    for _ in range(steps):
        mixed = rng.standard_normal((batch, chn)).astype(np.float32)
        gate = rng.standard_normal((batch, hv * dv)).astype(np.float32)
        bl = rng.standard_normal((batch, hv)).astype(np.float32)
        al = rng.standard_normal((batch, hv)).astype(np.float32)
        out = ops.recurrent_layer_step_(ws, T(mixed), T(w), T(gate), T(bl), T(al), T(dt), T(ssm),
                                        T(nw), key_heads=hk, key_dimension=dk, epsilon=1e-6,
                                        out_dtype=out_dtype)
        outs.append(out.float().cpu().numpy())
    return outs, ws.delta_state.cpu().numpy(), ws.convolution_history.cpu().numpy()


@pytest.mark.parametrize("out_name", ["f32", "bf16"])
@pytest.mark.parametrize("batch,hk,hv,dk,dv,kernel", [(1, 16, 32, 128, 128, 4),
                                                      (2, 2, 4, 64, 96, 4),
                                                      (3, 1, 2, 256, 40, 4),
                                                      (1, 2, 6, 32, 48, 1)])
def test_recurrent_layer_step_one_launch_matches_three_launches(gpu, ops, override, out_name,
                                                                batch, hk, hv, dk, dv, kernel):
    """The one-launch step (one block per key head) performs the prep / GDN
    step / gated-norm arithmetic of the three-launch path in the same order,
    so the two agree bit for bit (outputs, state and history)."""
    import torch
    args = (ops, torch, gpu, 7 + hk * 3 + kernel, batch, hk, hv, dk, dv, kernel,
            _td(torch, out_name), 4)
    fused = _recurrent_run(*args)
    override("recurrent_unfused", 1)
    split = _recurrent_run(*args)
    for a, b in zip(fused[0], split[0]):
        assert np.array_equal(a, b)
    assert np.array_equal(fused[1], split[1])
    assert np.array_equal(fused[2], split[2])


def test_qwen35_recurrent_layer_numpy(gpu):
    K = _mod("qwen35_kernels")
    rng = np.random.default_rng(21)
    hk, hv, dk, dv = 4, 8, 64, 64
    state = (rng.standard_normal((hv, dv, dk)) * 0.1).astype(np.float32)
    s64 = state.astype(np.float64)
    q = rng.standard_normal((hk, dk)).astype(np.float32)
    k = rng.standard_normal((hk, dk)).astype(np.float32)
    v = rng.standard_normal((hv, dv)).astype(np.float32)
    bl, al, dt = (rng.standard_normal(hv).astype(np.float32) for _ in range(3))
    ssm = (-np.exp(rng.uniform(-1, 1, hv))).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, dv).astype(np.float32)
    gates = rng.standard_normal((hv, dv)).astype(np.float32)
    gated, qn, kn = K.qwen35_recurrent_layer(state, q, k, v, bl, al, dt, ssm, nw, gates, 1e-6)
    from oracle import gdn as G
    rq, rk = L.l2_normalize(q, 1e-6), L.l2_normalize(k, 1e-6)
    beta, g = L.recurrent_parameters(bl, al, dt, ssm)
    o = G.gdn_step(s64, rq, rk, v, beta, g)
    ref = L.gated_rms_norm(o, nw, gates, 1e-6)
    assert np.abs(gated - ref).max() <= 1e-4
    assert np.abs(qn - rq).max() <= 1e-5 and np.abs(kn - rk).max() <= 1e-5
    assert np.abs(state - s64).max() <= 1e-4


def test_split_query_gate(gpu, ops):
    import torch
    p = torch.arange(2 * 3 * 2 * 4, dtype=torch.float32, device=gpu).reshape(2, 24)
    q, g = ops.split_query_gate(p, query_heads=3, head_dimension=4)
    rq, rg = L.split_query_gate(p.cpu().numpy(), 3, 4)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(g.cpu().numpy(), rg)


# ------------------------------------------------ seeded random geometry

def _pick(rng, values):
    return values[int(rng.integers(len(values)))]


def _random_step_cases(n=24):
    rng = np.random.default_rng(9600)
    cases = []
    for i in range(n):
        dtype = _pick(rng, ["bf16", "f16", "bf16", "f32"])
        d = _pick(rng, [64, 128, 256, 128, 96])
        sections = _pick(rng, [s for s in ((11, 11, 10, 0), (16, 16, 16, 16), (8, 12, 12, 0),
                                           (4, 4, 2, 0), (10, 10, 10, 2))
                               if 2 * sum(s) <= d])
        b = int(rng.integers(1, 6))
        hkv = int(rng.integers(1, 4))
        hq = hkv * _pick(rng, [1, 2, 4, 8])
        cap = int(rng.integers(1, 2049))
        ragged = bool(b > 1 and rng.random() < 0.4)
        rows = (rng.integers(0, cap, b) if ragged else np.full(b, int(rng.integers(0, cap))))
        c = dict(seed=9600 + i, dtype=dtype, d=d, sections=sections, b=b, hkv=hkv, hq=hq,
                 cap=cap, rows=[int(x) for x in rows], ragged=ragged,
                 out32=bool(dtype != "f32" and rng.random() < 0.4))
        c["id"] = (f"step{i:02d}-{dtype}-d{d}-q{hq}kv{hkv}-B{b}-cap{cap}-R{sum(sections)}"
                   f"{'-ragged' if ragged else '-at%d' % rows[0]}{'-o32' if c['out32'] else ''}")
        cases.append(c)
    return cases


def _random_recurrent_step_cases(n=12):
    rng = np.random.default_rng(9650)
    cases = []
    for i in range(n):
        hk = int(rng.integers(1, 4))
        c = dict(seed=9650 + i, batch=int(rng.integers(1, 4)), hk=hk,
                 hv=hk * int(rng.integers(1, 4)), dk=_pick(rng, [32, 64, 128, 256, 40]),
                 dv=_pick(rng, [32, 48, 96, 128, 24]), kernel=_pick(rng, [4, 4, 3, 2, 1, 6]),
                 steps=int(rng.integers(2, 9)))
        c["id"] = (f"rstep{i:02d}-B{c['batch']}-hk{hk}hv{c['hv']}-k{c['dk']}v{c['dv']}"
                   f"-taps{c['kernel']}-x{c['steps']}")
        cases.append(c)
    return cases


STEP_CASES = _random_step_cases()
RSTEP_CASES = _random_recurrent_step_cases()


@pytest.mark.parametrize("c", STEP_CASES, ids=[c["id"] for c in STEP_CASES])
def test_random_attention_layer_step_against_oracle(gpu, ops, c):
    """Seeded random geometry (dtype, head dim, rotary sections, batch,
    heads, capacity, uniform or per-sequence rows, output dtype) of the
    fused attention-layer step against the oracle prologue and decode: key
    rows at the dtype's bar, value rows copied bit for bit, the gated
    output of each sequence over its rows 0 .. row, every other cache row
    untouched."""
    import torch
    print("random attention layer step:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, d, b, hq, hkv, cap, rows = (c["dtype"], c["d"], c["b"], c["hq"], c["hkv"], c["cap"],
                                    c["rows"])
    base, eps = 10000000.0, 1e-6
    kc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dt)
    vc = I.round_to(rng.standard_normal((cap, b, hkv, d)), dt)
    qg = I.round_to(rng.standard_normal((b, hq * 2 * d)) * 3, dt)
    k = I.round_to(rng.standard_normal((b, hkv * d)) * 3, dt)
    v = I.round_to(rng.standard_normal((b, hkv * d)), dt)
    qw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    KC, VC = _dev(torch, kc, dt, gpu), _dev(torch, vc, dt, gpu)
    bound = max(rows)
    out, n = ops.attention_layer_step_(
        _dev(torch, qg, dt, gpu), _dev(torch, k, dt, gpu), _dev(torch, v, dt, gpu),
        torch.from_numpy(qw).to(gpu), torch.from_numpy(kw).to(gpu), KC, VC, position=bound,
        positions=rows if c["ragged"] else None, sections=c["sections"], frequency_base=base,
        epsilon=eps, out_dtype=torch.float32 if c["out32"] else None)
    torch.cuda.synchronize()
    assert n == bound + 1 and tuple(out.shape) == (b, hq, d)
    assert out.dtype == (torch.float32 if c["out32"] else _td(torch, dt))
    rq, rg, rk, rv = L.attention_prologue(qg, k, v, qw, kw, eps, np.array(rows), c["sections"],
                                          base)
    tol = _tol(dt)
    got_k, got_v = _np(KC), _np(VC)
    worst = 0.0
    for bb, p in enumerate(rows):
        assert np.abs(got_k[p, bb] - rk[bb]).max() <= tol, (c["id"], bb)
        assert np.array_equal(got_v[p, bb], rv[bb]), (c["id"], bb)
        ref = A.attention_decode_twopass(rq[bb], got_k[:p + 1, bb], got_v[:p + 1, bb],
                                         hq // hkv, 1.0 / np.sqrt(d))
        ref = ref * (1.0 / (1.0 + np.exp(-rg[bb])))
        worst = max(worst, float(np.abs(_np(out[bb]) - ref).max()))
    print(f"  output {worst:.3g} (bar {tol:g})", flush=True)
    assert worst <= tol, (c["id"], worst)
    mask = np.ones((cap, b), bool)
    mask[rows, np.arange(b)] = False
    assert np.array_equal(got_k[mask], kc[mask]) and np.array_equal(got_v[mask], vc[mask])


@pytest.mark.parametrize("c", RSTEP_CASES, ids=[c["id"] for c in RSTEP_CASES])
def test_random_recurrent_layer_step_against_oracle(gpu, ops, c):
    """Seeded random geometry (batch, head counts, head dims, convolution
    taps, number of tokens) of the recurrent-layer step against the fp64
    token chain: output and state 1e-4, convolution history bit for bit."""
    import torch
    print("random recurrent layer step:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    batch, hk, hv, dk, dv, kernel = c["batch"], c["hk"], c["hv"], c["dk"], c["dv"], c["kernel"]
    eps = 1e-6
    chn = 2 * hk * dk + hv * dv
    w = (rng.standard_normal((kernel, chn)) * 0.5).astype(np.float32)
    dt = rng.standard_normal(hv).astype(np.float32)
    ssm = (-np.exp(rng.uniform(-1, 1, hv))).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, dv).astype(np.float32)
    ws = ops.initialize_recurrent_workspace(batch_size=batch, convolution_kernel=kernel,
                                            convolution_channels=chn, value_heads=hv,
                                            value_dimension=dv, key_dimension=dk)
    hist = np.zeros((batch, kernel - 1, chn))
    state = np.zeros((batch, hv, dv, dk))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(gpu)  # noqa: E731
    worst = 0.0
    for _ in range(c["steps"]):
        mixed = rng.standard_normal((batch, chn)).astype(np.float32)
        gate = rng.standard_normal((batch, hv * dv)).astype(np.float32)
        bl = rng.standard_normal((batch, hv)).astype(np.float32)
        al = rng.standard_normal((batch, hv)).astype(np.float32)
        out = ops.recurrent_layer_step_(ws, T(mixed), T(w), T(gate), T(bl), T(al), T(dt), T(ssm),
                                        T(nw), key_heads=hk, key_dimension=dk, epsilon=eps)
        ref, hist = L.recurrent_layer_step(mixed, w, hist, gate, bl, al, dt, ssm, nw, state,
                                           key_heads=hk, key_dim=dk, value_heads=hv,
                                           value_dim=dv, eps=eps)
        worst = max(worst, float(np.abs(out.cpu().numpy() - ref).max()))
    err_s = float(np.abs(ws.delta_state.cpu().numpy() - state).max())
    print(f"  output {worst:.3g}, state {err_s:.3g} (bar 1e-4)", flush=True)
    assert worst <= 1e-4 and err_s <= 1e-4, (c["id"], worst, err_s)
    assert np.array_equal(ws.convolution_history.cpu().numpy(), hist.astype(np.float32))


def _random_norm_cases(n=24):
    rng = np.random.default_rng(9700)
    widths = [int(rng.integers(1, 129)), int(rng.integers(129, 257)),
              int(rng.integers(257, 513)), int(rng.integers(513, 1200))]
    cases = []
    for i in range(n):
        c = dict(seed=9700 + i, dtype=_pick(rng, ["f32", "bf16", "f16"]),
                 n=widths[i % 4] if i < 8 else int(rng.integers(1, 1200)),
                 rows=int(rng.integers(1, 70)), eps=_pick(rng, [1e-6, 1e-5]))
        c["id"] = f"norm{i:02d}-{c['dtype']}-n{c['n']}-rows{c['rows']}"
        cases.append(c)
    return cases


NORM_CASES = _random_norm_cases()


@pytest.mark.parametrize("c", NORM_CASES, ids=[c["id"] for c in NORM_CASES])
def test_random_row_norms_against_oracle(gpu, ops, c):
    """Seeded random row widths (every width class the kernel dispatches on:
    up to 128, 256 and 512 values per row held in registers, wider rows in a
    strided loop), row counts and dtypes of the L2, RMS and gated RMS norms
    against the oracle, at the dtype's bar plus one unit in the last place
    of the output's format (|2^-7 x| for bf16, |2^-10 x| for fp16)."""
    import torch
    print("random row norms:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, n = c["dtype"], c["n"]
    x = I.round_to(rng.standard_normal((c["rows"], n)) * 2.0, dt)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    gt = I.round_to(rng.standard_normal((c["rows"], n)), dt)
    X, G_ = _dev(torch, x, dt, gpu), _dev(torch, gt, dt, gpu)
    W = torch.from_numpy(w).to(gpu)
    tol = _tol(dt)
    # normalised rows reach |4-8| (RMS x weight) and past 16 (x silu(gate)),
    # where one unit in the last place of bf16 is 2^-5 to 2^-3: the bar is
    # the dtype's tolerance plus one unit in the last place of the output
    ulp = {"f32": 0.0, "f16": 2.0 ** -10, "bf16": 2.0 ** -7}[dt]

    def err(got, ref):
        return float((np.abs(_np(got) - ref) - ulp * np.abs(ref)).max())
    errs = (err(ops.rms_norm(X, W, c["eps"]), L.rms_norm(x, w, c["eps"])),
            err(ops.l2_normalize(X, c["eps"]), L.l2_normalize(x, c["eps"])),
            err(ops.recurrent_gate(X, W, G_, c["eps"]), L.gated_rms_norm(x, w, gt, c["eps"])))
    print("  beyond one output ulp: rms %.3g, l2 %.3g, gated %.3g (bar %g)" % (*errs, tol),
          flush=True)
    assert max(errs) <= tol, (c["id"], errs)


def _random_conv_cases(n=12):
    rng = np.random.default_rng(9750)
    return [dict(seed=9750 + i, kernel=int(rng.integers(1, 7)), batch=int(rng.integers(1, 5)),
                 channels=int(rng.integers(1, 9000)),
                 id=f"conv{i:02d}") for i in range(n)]


CONV_CASES = _random_conv_cases()
for _c in CONV_CASES:
    _c["id"] += f"-taps{_c['kernel']}-B{_c['batch']}-C{_c['channels']}"


@pytest.mark.parametrize("c", CONV_CASES, ids=[c["id"] for c in CONV_CASES])
def test_random_conv_step_against_oracle(gpu, ops, c):
    """Seeded random taps (1-6), batch and channel counts of the depthwise
    causal convolution step: output at 1e-4, the history shift bit for
    bit."""
    import torch
    print("random conv step:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    b, ch, kernel = c["batch"], c["channels"], c["kernel"]
    cur = rng.standard_normal((b, ch)).astype(np.float32)
    w = rng.standard_normal((kernel, ch)).astype(np.float32)
    hist = rng.standard_normal((b, kernel - 1, ch)).astype(np.float32)
    H = torch.from_numpy(hist).to(gpu)
    out = ops.causal_convolution_step_(torch.from_numpy(cur).to(gpu),
                                       torch.from_numpy(w).to(gpu), H)
    ref, new_hist = L.conv_step(cur, w, hist)
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-4, c["id"]
    assert np.array_equal(H.cpu().numpy(), new_hist.astype(np.float32)), c["id"]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_many_row_norms_equal_one_row_per_wave(gpu, dtype):
    """Calls of many rows of at most 128 values run four rows per wave; the
    same rows in calls of fewer rows run one row per wave.  The per-row
    arithmetic is the same, so every mode gives the same bits either way."""
    import torch
    ops_mod = _mod("_ops")
    lib = _mod("_lib")
    rng = np.random.default_rng(31)
    rows, n = 8192 + 3, 128
    x = _dev(torch, I.round_to(rng.standard_normal((rows, n)) * 2.0, dtype), dtype, gpu)
    g = _dev(torch, I.round_to(rng.standard_normal((rows, n)), dtype), dtype, gpu)
    w = torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float32)).to(gpu)
    for mode in (lib.NORM_L2, lib.NORM_RMS, lib.NORM_RMS_GATE):
        kw = dict(mode=mode, eps=1e-6, n=n)
        if mode != lib.NORM_L2:
            kw["weight"] = w
        if mode == lib.NORM_RMS_GATE:
            kw["gate"] = g
        whole = ops_mod.row_norm(x, rows=rows, **kw)
        parts = []
        for r0 in range(0, rows, 2048):
            r1 = min(rows, r0 + 2048)
            kp = dict(kw)
            if mode == lib.NORM_RMS_GATE:
                kp["gate"] = g[r0:r1]
            parts.append(ops_mod.row_norm(x[r0:r1], rows=r1 - r0, **kp))
        torch.cuda.synchronize()
        bits = torch.int32 if dtype == "f32" else torch.int16
        assert torch.equal(whole.view(bits), torch.cat(parts).view(bits)), mode
