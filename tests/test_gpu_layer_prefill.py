"""GPU parity of the chunked Qwen3.5 layer prefill (the caller that runs a
chunk of tokens through the attention / recurrent layer in a few launches,
where the reference runs one token at a time) against the fp64
token-sequential oracle (oracle/layer.py) and against the device's own
per-token path.

Tolerances: bf16 results 2e-2; the recurrent chunk (fp32 end to end, as
the reference's chain) 1e-4 on output and state against the unrounded fp64
chain; its fp32 prep outputs 1e-5 (fp32 arithmetic); with the opt-in bf16
q / k / v operands, the GDN state 1e-4 when the oracle is fed the device's
own bf16 q / k / v and 2e-3 when it rounds its own (a value on a bf16
rounding boundary may round to the neighbouring bf16 on one side), the
output 2e-2; pure copies (value rows, convolution history) bit-exact."""

import importlib

import numpy as np
import pytest

from oracle import gdn as G
from oracle import inputs as I
from oracle import layer as L

pytestmark = pytest.mark.gpu


def _mod(name):
    return importlib.import_module("alpacca-open-sourced-by-jt_amd." + name)


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.fixture(scope="module")
def ops(gpu):
    return _mod("qwen35_rocm_ops").Qwen35RocmOps()


def _bf16(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(torch.bfloat16)


def _f32(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


# ------------------------------------------------------- attention layer

@pytest.mark.parametrize("hq,hkv,d,sections,prefix,tokens,batch,bi", [
    (4, 2, 64, (11, 11, 10, 0), 5, 37, 1, 0),          # small, ragged chunk
    (16, 2, 256, (11, 11, 10, 0), 700, 130, 2, 1),     # Qwen3.5 geometry, second sequence
    (8, 8, 128, (16, 16, 16, 16), 0, 64, 1, 0),        # empty prefix, all four sections
])
def test_attention_layer_prefill_matches_token_chain(gpu, ops, hq, hkv, d, sections, prefix,
                                                     tokens, batch, bi):
    import torch
    rng = np.random.default_rng(hq * 1000 + d + prefix)
    base, eps, cap = 10000000.0, 1e-6, prefix + tokens + 8
    r = lambda a: I.round_to(a, "bf16")  # noqa: E731
    kc0 = np.zeros((cap, batch, hkv, d))
    vc0 = np.zeros((cap, batch, hkv, d))
    kc0[:prefix] = r(rng.standard_normal((prefix, batch, hkv, d)))
    vc0[:prefix] = r(rng.standard_normal((prefix, batch, hkv, d)))
    qg = r(rng.standard_normal((tokens, hq * 2 * d)) * 3)
    k = r(rng.standard_normal((tokens, hkv * d)) * 3)
    v = r(rng.standard_normal((tokens, hkv * d)))
    qw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    QW, KW = _f32(torch, qw, gpu), _f32(torch, kw, gpu)
    # chunk path
    KC, VC = _bf16(torch, kc0, gpu), _bf16(torch, vc0, gpu)
    out, nxt = ops.attention_layer_prefill_(
        _bf16(torch, qg, gpu), _bf16(torch, k, gpu), _bf16(torch, v, gpu), QW, KW, KC, VC,
        position=prefix, batch_index=bi, sections=sections, frequency_base=base, epsilon=eps)
    torch.cuda.synchronize()
    assert nxt == prefix + tokens and tuple(out.shape) == (tokens, hq, d)
    # the device's own token-by-token path on a copy of the caches
    KT, VT = _bf16(torch, kc0, gpu), _bf16(torch, vc0, gpu)
    steps = []
    for t in range(tokens):
        rows = slice(t, t + 1)
        qg_b = np.zeros((batch, hq * 2 * d))
        k_b = np.zeros((batch, hkv * d))
        v_b = np.zeros((batch, hkv * d))
        qg_b[bi], k_b[bi], v_b[bi] = qg[rows][0], k[rows][0], v[rows][0]
        pos = np.full(batch, -1, dtype=np.int32)   # other sequences: no cache write
        pos[bi] = prefix + t
        q_dev, g_dev = _mod("_ops").attention_prologue(
            _bf16(torch, qg_b, gpu).reshape(batch, hq, 2 * d), _bf16(torch, k_b, gpu),
            _bf16(torch, v_b, gpu), QW, KW, KT, VT, positions=torch.from_numpy(pos).to(gpu),
            sections=sections, frequency_base=base, eps=eps)
        o = ops.online_attention(q_dev, KT, VT, length=prefix + t + 1, gate=g_dev)
        steps.append(_np(o[bi]))
    torch.cuda.synchronize()
    # same prologue kernel, same rows: the caches agree bit for bit
    assert torch.equal(KC.view(torch.int16), KT.view(torch.int16))
    assert torch.equal(VC.view(torch.int16), VT.view(torch.int16))
    assert np.array_equal(_np(VC)[prefix:prefix + tokens, bi], v.reshape(tokens, hkv, d))
    untouched = np.ones(batch, bool)
    untouched[bi] = False
    assert np.array_equal(_np(KC)[:, untouched], kc0[:, untouched])
    assert np.abs(_np(out) - np.stack(steps)).max() <= 2e-2
    # fp64 token-sequential oracle (bf16 cache rows)
    kco, vco = kc0[:, bi].copy(), vc0[:, bi].copy()
    ref = L.attention_layer_prefill(qg, k, v, qw, kw, eps, prefix, sections, base, kco, vco,
                                    round_rows=r)
    assert np.abs(_np(out) - ref).max() <= 2e-2
    assert np.abs(_np(KC)[:prefix + tokens, bi] - kco[:prefix + tokens]).max() <= 2e-2


@pytest.mark.parametrize("hq,hkv,d,prefix,tokens,batch,bi,dtype,sec", [
    (16, 2, 256, 300, 130, 2, 1, "bf16", (11, 11, 10, 0)),
    (8, 2, 128, 0, 70, 1, 0, "f16", (11, 11, 10, 0)),
    (4, 2, 64, 40, 33, 1, 0, "f32", (11, 11, 10, 0)),
    (8, 2, 128, 17, 1, 1, 0, "bf16", (16, 16, 16, 16)),     # 2 R = D, one token
    (4, 2, 64, 90, 45, 3, 2, "bf16", (8, 8, 8, 8)),         # 2 R = D at D = 64
    (16, 2, 256, 2500, 384, 1, 0, "bf16", (11, 11, 10, 0)),  # long prefix, shared kernel
    (16, 2, 256, 0, 1000, 1, 0, "f16", (24, 20, 20, 0)),    # R = 64, multi-round pairs
    (8, 2, 128, 30, 50, 1, 0, "bf16", (10, 10, 10, 0)),     # R = 30: query buffer only
])
def test_attention_layer_prefill_equals_prologue_then_gated_prefill(gpu, hq, hkv, d, prefix,
                                                                    tokens, batch, bi, dtype,
                                                                    sec):
    """alpx_attention_layer_prefill in both of its forms gives the bits of
    alpx_attention_prologue_chunk (gate copied) + alpx_prefill_causal_gated:
    output and both caches.  The query-buffer form writes the query rows
    and has the prefill read the gate in place from the joint projection
    (row stride 2 D; fp32 runs the split-K fallback, whose combine applies
    the gate); the fused form (fp16 / bf16, rotary pairs in whole groups of
    32) has the prefill form the query rows from the joint projection
    itself, with the prologue's RMS reduction order and rotation table."""
    import torch
    P = _mod("_ops")
    Lib = _mod("_lib")
    td = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    rng = np.random.default_rng(hq + d + prefix)
    cap = prefix + tokens + 5
    base, eps = 1e6, 1e-6
    t = lambda a: torch.from_numpy(I.round_to(a, dtype).astype(np.float32)).to(gpu).to(td)  # noqa: E731
    kc0 = t(rng.standard_normal((cap, batch, hkv, d)))
    vc0 = t(rng.standard_normal((cap, batch, hkv, d)))
    qg = t(rng.standard_normal((tokens, hq, 2 * d)) * 3)
    k = t(rng.standard_normal((tokens, hkv, d)) * 3)
    v = t(rng.standard_normal((tokens, hkv, d)))
    qw = torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(gpu)
    kw = torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(gpu)
    KB, VB = kc0.clone(), vc0.clone()
    q, g = P.attention_prologue_chunk(qg, k, v, qw, kw, KB, VB, batch_index=bi, position=prefix,
                                      sections=sec, frequency_base=base, eps=eps)
    out_b = P.prefill(q, KB[:, bi], VB[:, bi], pos0=prefix, kv_tokens=prefix + tokens,
                      k_pos_stride=batch * hkv * d, v_pos_stride=batch * hkv * d, gate=g)
    torch.cuda.synchronize()
    assert torch.equal(g, qg[:, :, d:])  # the copied gate is the joint row's second half
    fusable = dtype != "f32" and sum(sec) % 32 == 0
    for fused in (None, False, True):
        KA, VA = kc0.clone(), vc0.clone()
        call = lambda: P.attention_layer_prefill(  # noqa: E731
            qg, k, v, qw, kw, KA, VA, batch_index=bi, position=prefix, sections=sec,
            frequency_base=base, eps=eps, fused_query=fused)
        if fused and not fusable:
            with pytest.raises(Lib.AlpxUnsupported, match="without query_out"):
                call()
            # refused before any launch: the caches are untouched
            assert torch.equal(KA, kc0) and torch.equal(VA, vc0)
            continue
        out_a = call()
        torch.cuda.synchronize()
        assert torch.equal(KA, KB) and torch.equal(VA, VB), fused
        assert torch.equal(out_a, out_b), fused


def test_attention_layer_prefill_cache_of_2gib_or_more(gpu, ops):
    """A chunk over caches of 2 GiB per tensor (16 sequences x 131072 rows of
    2 x 256 bf16): the MFMA prefill's 32-bit row offsets do not reach, so
    the form without a query buffer refuses before any launch and the call
    runs the query-buffer form on the split-K prefill with a workspace.  Its
    output agrees with the same chunk over a batch-1 copy of the sequence
    (MFMA kernels), the written rows bit for bit, and the other sequences
    stay untouched."""
    import torch
    hq, hkv, d, cache_batch, cap, tokens, bi = 16, 2, 256, 16, 131072, 64, 5
    assert cap * cache_batch * hkv * d * 2 == 1 << 31
    pos = cap - tokens
    gen = torch.Generator(device=gpu).manual_seed(11)
    seq_k = torch.randn((pos, hkv, d), device=gpu, generator=gen).to(torch.bfloat16)
    seq_v = torch.randn((pos, hkv, d), device=gpu, generator=gen).to(torch.bfloat16)
    KC = torch.zeros((cap, cache_batch, hkv, d), dtype=torch.bfloat16, device=gpu)
    VC = torch.zeros_like(KC)
    KC[:pos, bi] = seq_k
    VC[:pos, bi] = seq_v
    KS = torch.zeros((cap, 1, hkv, d), dtype=torch.bfloat16, device=gpu)
    VS = torch.zeros_like(KS)
    KS[:pos, 0] = seq_k
    VS[:pos, 0] = seq_v
    del seq_k, seq_v
    qg = (torch.randn((tokens, hq * 2 * d), device=gpu, generator=gen) * 3).to(torch.bfloat16)
    k = (torch.randn((tokens, hkv * d), device=gpu, generator=gen) * 3).to(torch.bfloat16)
    v = torch.randn((tokens, hkv * d), device=gpu, generator=gen).to(torch.bfloat16)
    w = torch.linspace(0.5, 1.5, d, device=gpu)
    kwargs = dict(position=pos, sections=(11, 11, 10, 0), frequency_base=1e7, epsilon=1e-6)
    big, nxt = ops.attention_layer_prefill_(qg, k, v, w, w, KC, VC, batch_index=bi, **kwargs)
    small, _ = ops.attention_layer_prefill_(qg, k, v, w, w, KS, VS, batch_index=0, **kwargs)
    torch.cuda.synchronize()
    assert nxt == cap
    assert torch.equal(KC[pos:, bi], KS[pos:, 0]) and torch.equal(VC[pos:, bi], VS[pos:, 0])
    assert (big.float() - small.float()).abs().max().item() <= 2e-2
    others = [b for b in range(cache_batch) if b != bi]
    assert KC[pos - 8:, others].abs().sum().item() == 0
    assert VC[:, others[:3]].abs().sum().item() == 0


def test_attention_layer_prefill_rejects_bad_shapes(gpu, ops):
    import torch
    KC = torch.zeros((16, 1, 2, 64), dtype=torch.bfloat16, device=gpu)
    VC = torch.zeros_like(KC)
    QW = torch.ones(64, device=gpu)
    qg = torch.zeros((4, 2 * 2 * 64), dtype=torch.bfloat16, device=gpu)
    k = torch.zeros((4, 2 * 64), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="capacity"):
        ops.attention_layer_prefill_(qg, k, k, QW, QW, KC, VC, position=13,
                                     sections=(11, 11, 10, 0), frequency_base=1e4, epsilon=1e-6)
    with pytest.raises(ValueError, match="batch_index"):
        ops.attention_layer_prefill_(qg, k, k, QW, QW, KC, VC, position=0, batch_index=1,
                                     sections=(11, 11, 10, 0), frequency_base=1e4, epsilon=1e-6)


# ------------------------------------------------------- recurrent layer

def _rec_inputs(rng, tokens, hk, hv, dk, dv, kernel):
    c = 2 * hk * dk + hv * dv
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    return dict(mixed=f(tokens, c), w=(f(kernel, c) * 0.5), hist=f(kernel - 1, c),
                gate=f(tokens, hv * dv), bl=f(tokens, hv), al=f(tokens, hv), dt=f(hv),
                ssm=(-np.exp(rng.uniform(-1, 1, hv))).astype(np.float32),
                nw=rng.uniform(0.5, 1.5, dv).astype(np.float32),
                s0=(f(hv, dv, dk) * 0.1))


@pytest.mark.parametrize("tokens,kernel,hk,hv,dk,dv", [
    (37, 4, 2, 4, 64, 32), (2, 4, 2, 4, 64, 32), (5, 1, 2, 4, 64, 32), (9, 6, 2, 4, 64, 32),
    (150, 4, 1, 2, 256, 128), (70, 3, 2, 4, 128, 40), (65, 2, 1, 3, 20, 36),
    (21, 4, 1, 2, 30, 16)])
def test_recurrent_prefill_prep_matches_oracle(gpu, tokens, kernel, hk, hv, dk, dv):
    # conv + SiLU over the chunk continuing the history, split, L2 norm,
    # beta / decay (fp32 outputs), and the history moved on; kernels of up
    # to 4 taps with head dims that are multiples of 4 take the tiled
    # kernel (token tiles of 64, partial last tile), the rest (6 taps,
    # dk = 30) the per-wave kernel
    import torch
    P = _mod("_ops")
    rng = np.random.default_rng(tokens * 10 + kernel)
    eps = 1e-6
    x = _rec_inputs(rng, tokens, hk, hv, dk, dv, kernel)
    H = _f32(torch, x["hist"], gpu) if kernel > 1 else None
    q, k, v, beta, g = P.recurrent_prefill_prep(
        _f32(torch, x["mixed"], gpu), _f32(torch, x["w"], gpu), H, _f32(torch, x["bl"], gpu),
        _f32(torch, x["al"], gpu), _f32(torch, x["dt"], gpu), _f32(torch, x["ssm"], gpu),
        key_heads=hk, key_dim=dk, value_heads=hv, value_dim=dv, eps=eps,
        qkv_dtype=torch.float32)
    hist = x["hist"].astype(np.float64)[None]
    w = hk * dk
    for t in range(tokens):
        act, hist = L.conv_step(x["mixed"][t:t + 1], x["w"], hist, apply_silu=True)
        assert np.abs(_np(q[t]) - L.l2_normalize(act[0, :w].reshape(hk, dk), eps)).max() <= 1e-5
        assert np.abs(_np(k[t]) - L.l2_normalize(act[0, w:2 * w].reshape(hk, dk),
                                                 eps)).max() <= 1e-5
        assert np.abs(_np(v[t]) - act[0, 2 * w:].reshape(hv, dv)).max() <= 1e-5
    rb, rg = L.recurrent_parameters(x["bl"], x["al"], x["dt"], x["ssm"])
    assert np.abs(_np(beta) - rb).max() <= 1e-6 and np.abs(_np(g) - rg).max() <= 1e-5
    if kernel > 1:
        assert np.array_equal(H.cpu().numpy(), hist[0].astype(np.float32))


@pytest.mark.parametrize("tokens,hk,hv,d,layout,qkv", [
    (70, 2, 4, 64, "kc", "f32"), (130, 1, 2, 128, "kc", "f32"), (65, 1, 1, 256, "kc", "f32"),
    (100, 2, 4, 128, "ck", "f32"), (37, 2, 4, 128, "kc", "bf16")])
def test_recurrent_prefill_prep_four_taps_equal_dims(gpu, tokens, hk, hv, d, layout, qkv):
    # 4-tap convolution with equal key / value head dims (the Qwen3.5
    # shapes) through the tiled kernel, for weights laid out [K, C] (tap rows
    # of consecutive channels) and [C, K], fp32 and bf16 outputs
    import torch
    P = _mod("_ops")
    rng = np.random.default_rng(tokens * 3 + d)
    eps, kernel = 1e-6, 4
    x = _rec_inputs(rng, tokens, hk, hv, d, d, kernel)
    w_dev = _f32(torch, x["w"], gpu) if layout == "kc" else _f32(torch, x["w"].T.copy(), gpu)
    H = _f32(torch, x["hist"], gpu)
    td = torch.float32 if qkv == "f32" else torch.bfloat16
    q, k, v, beta, g = P.recurrent_prefill_prep(
        _f32(torch, x["mixed"], gpu), w_dev, H, _f32(torch, x["bl"], gpu),
        _f32(torch, x["al"], gpu), _f32(torch, x["dt"], gpu), _f32(torch, x["ssm"], gpu),
        key_heads=hk, key_dim=d, value_heads=hv, value_dim=d, eps=eps, qkv_dtype=td,
        weight_layout=layout)
    tol = 1e-5 if qkv == "f32" else 1e-2
    hist = x["hist"].astype(np.float64)[None]
    w = hk * d
    for t in range(tokens):
        act, hist = L.conv_step(x["mixed"][t:t + 1], x["w"], hist, apply_silu=True)
        assert np.abs(_np(q[t]) - L.l2_normalize(act[0, :w].reshape(hk, d), eps)).max() <= tol
        assert np.abs(_np(k[t]) - L.l2_normalize(act[0, w:2 * w].reshape(hk, d), eps)).max() <= tol
        assert np.abs(_np(v[t]) - act[0, 2 * w:].reshape(hv, d)).max() <= tol * (1 if qkv == "f32" else 10)
    rb, rg = L.recurrent_parameters(x["bl"], x["al"], x["dt"], x["ssm"])
    assert np.abs(_np(beta) - rb).max() <= 1e-6 and np.abs(_np(g) - rg).max() <= 1e-5
    assert np.array_equal(H.cpu().numpy(), hist[0].astype(np.float32))


def _recurrent_prefill_vs_chain(ops, gpu, tokens, hk, hv, dk, dv, operand_dtype, seed=None,
                                kernel=4):
    # the chunk (prep -> chunked GDN -> gated norm) of the second sequence of
    # a batch-2 workspace, from a nonzero state and history, and the fp64
    # token-sequential chain; returns (device output, device state,
    # reference output, reference state), the oracle rounding q / k / v to
    # bf16 where the device is asked to
    import torch
    rng = np.random.default_rng(tokens + hk + dk if seed is None else seed)
    eps, bi = 1e-6, 1
    x = _rec_inputs(rng, tokens, hk, hv, dk, dv, kernel)
    c = 2 * hk * dk + hv * dv
    ws = ops.initialize_recurrent_workspace(batch_size=2, convolution_kernel=kernel,
                                            convolution_channels=c, value_heads=hv,
                                            value_dimension=dv, key_dimension=dk)
    ws.convolution_history[bi].copy_(_f32(torch, x["hist"], gpu))
    ws.delta_state[bi].copy_(_f32(torch, x["s0"], gpu))
    out = ops.recurrent_layer_prefill_(
        ws, _f32(torch, x["mixed"], gpu), _f32(torch, x["w"], gpu), _f32(torch, x["gate"], gpu),
        _f32(torch, x["bl"], gpu), _f32(torch, x["al"], gpu), _f32(torch, x["dt"], gpu),
        _f32(torch, x["ssm"], gpu), _f32(torch, x["nw"], gpu), key_heads=hk,
        key_dimension=dk, epsilon=eps, batch_index=bi, operand_dtype=operand_dtype)
    torch.cuda.synchronize()
    rounded = operand_dtype == torch.bfloat16 and dk in (64, 128, 256) and dv % 16 == 0
    state = x["s0"].astype(np.float64)
    ref, hist = L.recurrent_layer_prefill(
        x["mixed"], x["w"], x["hist"], x["gate"], x["bl"], x["al"], x["dt"], x["ssm"], x["nw"],
        state, key_heads=hk, key_dim=dk, value_heads=hv, value_dim=dv, eps=eps,
        round_qkv=(lambda a: I.round_to(a, "bf16")) if rounded else None)
    assert tuple(out.shape) == (tokens, hv * dv)
    assert np.array_equal(ws.convolution_history[bi].cpu().numpy(), hist.astype(np.float32))
    # the other sequence is untouched
    assert not ws.delta_state[0].any() and not ws.convolution_history[0].any()
    return _np(out), ws.delta_state[bi].cpu().numpy(), ref, state


@pytest.mark.parametrize("tokens,hk,hv,dk,dv", [(200, 16, 32, 128, 128), (1024, 16, 32, 128, 128),
                                                (70, 2, 4, 64, 64), (130, 1, 2, 256, 128),
                                                (33, 2, 2, 40, 24)])
def test_recurrent_layer_prefill_matches_token_chain(gpu, ops, tokens, hk, hv, dk, dv):
    # the fp32 chunk against the unrounded fp64 token chain at the fp32 bar:
    # the chunked GDN takes q / k / v as hi + lo bf16 operands (head dims
    # 64 / 128 / 256), (40, 24) runs it token by token; (1024, C5 heads) is
    # a full C5-geometry chunk
    out, state, ref, ref_state = _recurrent_prefill_vs_chain(ops, gpu, tokens, hk, hv, dk, dv,
                                                              None)
    assert np.abs(out - ref).max() <= 1e-4
    assert np.abs(state - ref_state).max() <= 1e-4


@pytest.mark.parametrize("tokens,hk,hv,dk,dv", [(200, 16, 32, 128, 128), (70, 2, 4, 64, 64)])
def test_recurrent_layer_prefill_bf16_operands(gpu, ops, tokens, hk, hv, dk, dv):
    # the opt-in bf16 q / k / v operands: against the chain whose oracle
    # rounds its own q / k / v to bf16, output 2e-2, state 2e-3 (a value on
    # a rounding boundary may land on the neighbouring bf16)
    import torch
    out, state, ref, ref_state = _recurrent_prefill_vs_chain(ops, gpu, tokens, hk, hv, dk, dv,
                                                              torch.bfloat16)
    assert np.abs(out - ref).max() <= 2e-2
    assert np.abs(state - ref_state).max() <= 2e-3


def test_recurrent_prefill_state_with_device_qkv(gpu):
    # C5 geometry: feed the oracle the device's own bf16 q / k / v, so the
    # chunked recurrence alone is compared -- state to 1e-4 over 300 tokens
    import torch
    P = _mod("_ops")
    rng = np.random.default_rng(5)
    tokens, hk, hv, dk, dv, kernel, eps = 300, 16, 32, 128, 128, 4, 1e-6
    x = _rec_inputs(rng, tokens, hk, hv, dk, dv, kernel)
    q, k, v, beta, g = P.recurrent_prefill_prep(
        _f32(torch, x["mixed"], gpu), _f32(torch, x["w"], gpu), _f32(torch, x["hist"], gpu),
        _f32(torch, x["bl"], gpu), _f32(torch, x["al"], gpu), _f32(torch, x["dt"], gpu),
        _f32(torch, x["ssm"], gpu), key_heads=hk, key_dim=dk, value_heads=hv, value_dim=dv,
        eps=eps, qkv_dtype=torch.bfloat16)
    S = _f32(torch, x["s0"], gpu)[None].contiguous()
    o = P.gdn_chunk(S, q[None], k[None], v[None], beta[None], g[None],
                    out_dtype=torch.float32)
    torch.cuda.synchronize()
    s64 = x["s0"].astype(np.float64)
    ro = G.gdn_scan(s64, _np(q), _np(k), _np(v), _np(beta), _np(g))
    assert np.abs(S[0].cpu().numpy() - s64).max() <= 1e-4
    assert np.abs(_np(o[0]) - np.asarray(ro)).max() <= 2e-2


# ------------------------------------------------ seeded random geometry

def _pick(rng, values):
    return values[int(rng.integers(len(values)))]


def _random_attention_layer_cases(n=16):
    rng = np.random.default_rng(9400)
    cases = []
    for i in range(n):
        dtype = _pick(rng, ["bf16", "f16", "bf16", "f32"])
        d = _pick(rng, [64, 128, 256, 128, 96])
        sec = _pick(rng, [s for s in ((11, 11, 10, 0), (16, 16, 16, 16), (8, 12, 12, 0),
                                      (24, 20, 20, 0), (5, 5, 6, 0), (10, 10, 10, 2))
                          if sum(s) <= d // 2])
        hkv = int(rng.integers(1, 4))
        hq = hkv * _pick(rng, [1, 2, 4, 8])
        tokens = int(rng.integers(1, 161))
        prefix = int(rng.integers(0, 601))
        batch = int(rng.integers(1, 4))
        c = dict(seed=9400 + i, dtype=dtype, d=d, sec=sec, hkv=hkv, hq=hq, tokens=tokens,
                 prefix=prefix, batch=batch, bi=int(rng.integers(batch)))
        c["id"] = (f"att{i:02d}-{dtype}-d{d}-q{hq}kv{hkv}-R{sum(sec)}-T{tokens}at{prefix}"
                   f"-B{batch}s{c['bi']}")
        cases.append(c)
    return cases


def _random_recurrent_cases(n=12):
    rng = np.random.default_rng(9450)
    cases = []
    for i in range(n):
        dk = _pick(rng, [64, 128, 256, 128, 40])
        dv = _pick(rng, [32, 64, 128, 256, 24])
        hk = int(rng.integers(1, 4))
        hv = hk * int(rng.integers(1, 4))
        tokens = max(1, min(int(rng.integers(1, 301)), 1200 // hv))
        c = dict(seed=9450 + i, dk=dk, dv=dv, hk=hk, hv=hv, tokens=tokens,
                 kernel=_pick(rng, [4, 4, 3, 2]))
        c["id"] = f"rec{i:02d}-k{dk}v{dv}-hk{hk}hv{hv}-T{tokens}-taps{c['kernel']}"
        cases.append(c)
    return cases


ATT_CASES = _random_attention_layer_cases()
REC_CASES = _random_recurrent_cases()


@pytest.mark.parametrize("c", ATT_CASES, ids=[c["id"] for c in ATT_CASES])
def test_random_attention_layer_prefill_against_token_chain(gpu, ops, c):
    """Seeded random geometry (dtype, head dim, rotary sections, heads,
    chunk, prefix, batch, sequence) of the chunked attention layer against
    the fp64 token-sequential oracle: gated output at the dtype's bar, the
    appended key rows within it, value rows copied bit for bit, the other
    sequences' rows untouched."""
    import torch
    print("random attention layer prefill:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, d, hq, hkv, T, P0, B, bi = (c["dtype"], c["d"], c["hq"], c["hkv"], c["tokens"],
                                    c["prefix"], c["batch"], c["bi"])
    td = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    r = lambda a: I.round_to(a, dt).astype(np.float64)  # noqa: E731
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(gpu).to(td)  # noqa: E731
    base, eps, cap = 1e6, 1e-6, P0 + T + 3
    kc0 = np.zeros((cap, B, hkv, d))
    vc0 = np.zeros((cap, B, hkv, d))
    kc0[:P0] = r(rng.standard_normal((P0, B, hkv, d)))
    vc0[:P0] = r(rng.standard_normal((P0, B, hkv, d)))
    qg = r(rng.standard_normal((T, hq * 2 * d)) * 3)
    k = r(rng.standard_normal((T, hkv * d)) * 3)
    v = r(rng.standard_normal((T, hkv * d)))
    qw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, d).astype(np.float32)
    KC, VC = dev(kc0), dev(vc0)
    out, nxt = ops.attention_layer_prefill_(
        dev(qg), dev(k), dev(v), _f32(torch, qw, gpu), _f32(torch, kw, gpu), KC, VC,
        position=P0, batch_index=bi, sections=c["sec"], frequency_base=base, epsilon=eps)
    torch.cuda.synchronize()
    assert nxt == P0 + T and tuple(out.shape) == (T, hq, d)
    kco, vco = kc0[:, bi].copy(), vc0[:, bi].copy()
    ref = L.attention_layer_prefill(qg, k, v, qw, kw, eps, P0, c["sec"], base, kco, vco,
                                    round_rows=None if dt == "f32" else r)
    tol = 1e-4 if dt == "f32" else 2e-2
    err = float(np.abs(_np(out) - ref).max())
    err_k = float(np.abs(_np(KC)[:P0 + T, bi] - kco[:P0 + T]).max())
    print(f"  output {err:.3g}, key rows {err_k:.3g} (bar {tol:g})", flush=True)
    assert err <= tol and err_k <= tol, (c["id"], err, err_k)
    assert np.array_equal(_np(VC)[P0:P0 + T, bi], v.reshape(T, hkv, d))
    others = np.arange(B) != bi
    assert np.array_equal(_np(KC)[:, others], kc0[:, others])
    assert np.array_equal(_np(VC)[:, others], vc0[:, others])


@pytest.mark.parametrize("c", REC_CASES, ids=[c["id"] for c in REC_CASES])
def test_random_recurrent_layer_prefill_against_token_chain(gpu, ops, c):
    """Seeded random geometry (head dims, head counts, chunk length,
    convolution taps) of the fp32 recurrent-layer chunk against the
    unrounded fp64 token chain at the fp32 bars (output and state 1e-4)."""
    print("random recurrent layer prefill:", c["id"], flush=True)
    out, state, ref, ref_state = _recurrent_prefill_vs_chain(
        ops, gpu, c["tokens"], c["hk"], c["hv"], c["dk"], c["dv"], None, seed=c["seed"],
        kernel=c["kernel"])
    err_o = float(np.abs(out - ref).max())
    err_s = float(np.abs(state - ref_state).max())
    print(f"  output {err_o:.3g}, state {err_s:.3g} (bar 1e-4)", flush=True)
    assert err_o <= 1e-4 and err_s <= 1e-4, (c["id"], err_o, err_s)
