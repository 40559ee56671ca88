"""GPU tests: the main entry points captured in a HIP graph and replayed.

Each case draws its geometry from a fixed seed, runs the call eagerly twice
on a side stream (sizing the facade's workspace), captures it with
``torch.cuda.graph``, then three times: writes fresh inputs into the
captured buffers, replays, keeps the replay's outputs and in-place states,
restores the states, runs the same call eagerly and requires the eager
results to equal the replay's bit for bit (the library records no memset,
allocation or host synchronisation, so a captured call must behave as the
eager one on whatever the buffers hold at replay time).
"""

import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _mod(name):
    return importlib.import_module("alpacca-open-sourced-by-jt_amd." + name)


@pytest.fixture(scope="module")
def ops(gpu):
    return _mod("qwen35_rocm_ops").Qwen35RocmOps()


def _pick(rng, values):
    return values[int(rng.integers(len(values)))]


def _cases(n_per_kind=3):
    rng = np.random.default_rng(9990)
    kinds = ("decode", "prefill", "gdn_chunk", "gdn_step", "attention_layer_step",
             "recurrent_layer_step")
    cases = []
    for kind in kinds:
        for i in range(n_per_kind):
            c = dict(kind=kind, seed=int(rng.integers(1 << 30)),
                     dtype=_pick(rng, ["bf16", "f16"] if kind != "recurrent_layer_step"
                                 else ["f32"]),
                     d=_pick(rng, [64, 128, 256]), hkv=int(rng.integers(1, 4)),
                     group=_pick(rng, [1, 2, 4, 8]), batch=int(rng.integers(1, 4)),
                     length=int(rng.integers(16, 1500)), tokens=int(rng.integers(1, 200)))
            if kind in ("gdn_chunk", "gdn_step"):
                c["dtype"] = _pick(rng, ["bf16", "f32"])
            c["id"] = (f"{kind}{i}-{c['dtype']}-d{c['d']}-kv{c['hkv']}x{c['group']}"
                       f"-B{c['batch']}-L{c['length']}-T{c['tokens']}")
            cases.append(c)
    return cases


CASES = _cases()


def _setup(torch, ops, gpu, c):
    """(step() -> outputs tuple, refresh(rng), mutable tensors) for case c."""
    td = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[c["dtype"]]
    g = torch.Generator(device=gpu).manual_seed(c["seed"])

    def rnd(shape, scale=1.0, dtype=td):
        return (torch.randn(shape, generator=g, device=gpu) * scale).to(dtype)

    d, hkv, B, L, T = c["d"], c["hkv"], c["batch"], c["length"], c["tokens"]
    hq = hkv * c["group"]
    kind = c["kind"]
    if kind == "decode":
        q, K, V = rnd((B, hq, d)), rnd((L, B, hkv, d)), rnd((L, B, hkv, d))
        gate = rnd((B, hq, d))
        lens = torch.full((B,), L, dtype=torch.int32, device=gpu)
        inputs = [q, K, V, gate]

        def step():
            return (ops.online_attention(q, K, V, length=L, seq_lens=lens, gate=gate),)

        def refresh(rng):
            for x in inputs:
                x.copy_(rnd(x.shape))
            lens.copy_(torch.from_numpy(rng.integers(1, L + 1, B).astype(np.int32)).to(gpu))
        return step, refresh, []
    if kind == "prefill":
        P = L
        K, V = rnd((P + T, B, hkv, d)), rnd((P + T, B, hkv, d))
        q, gate = rnd((T, hq, d)), rnd((T, hq, d))
        inputs = [q, K, V, gate]
        bi = B - 1

        def step():
            return (ops.attention_prefill(q, K, V, position=P, batch_index=bi, gate=gate),)

        def refresh(rng):
            for x in inputs:
                x.copy_(rnd(x.shape))
        return step, refresh, []
    if kind in ("gdn_chunk", "gdn_step"):
        hk, hv, dk, dv = hkv, hkv * min(c["group"], 2), d, _pick(np.random.default_rng(
            c["seed"]), [32, 64, 128])
        shape_t = (B, T) if kind == "gdn_chunk" else (B,)
        S = torch.randn((B, hv, dv, dk), generator=g, device=gpu) * 0.2

        def unit(shape):
            x = torch.randn(shape, generator=g, device=gpu)
            return (x / x.norm(dim=-1, keepdim=True)).to(td)
        q, k = unit(shape_t + (hk, dk)), unit(shape_t + (hk, dk))
        v = rnd(shape_t + (hv, dv))
        beta = torch.rand(shape_t + (hv,), generator=g, device=gpu)
        gdec = -torch.rand(shape_t + (hv,), generator=g, device=gpu) * 1.5

        def step():
            if kind == "gdn_chunk":
                return (ops.gated_delta_net_chunk_(S, q, k, v, beta, gdec),)
            return (ops.gated_delta_net_step_(S, q, k, v, beta, gdec),)

        def refresh(rng):
            q.copy_(unit(q.shape))
            k.copy_(unit(k.shape))
            v.copy_(rnd(v.shape))
            beta.copy_(torch.rand(beta.shape, generator=g, device=gpu))
            gdec.copy_(-torch.rand(gdec.shape, generator=g, device=gpu) * 1.5)
            S.copy_(torch.randn(S.shape, generator=g, device=gpu) * 0.2)
        return step, refresh, [S]
    if kind == "attention_layer_step":
        cap = L
        KC, VC = rnd((cap, B, hkv, d)), rnd((cap, B, hkv, d))
        qg, kk, vv = rnd((B, hq * 2 * d), 3.0), rnd((B, hkv * d), 3.0), rnd((B, hkv * d))
        qw = torch.rand(d, generator=g, device=gpu) + 0.5
        kw = torch.rand(d, generator=g, device=gpu) + 0.5
        positions = torch.zeros(B, dtype=torch.int32, device=gpu)
        sections = (11, 11, 10, 0) if d >= 64 else (4, 4, 2, 0)

        def step():
            out, _ = ops.attention_layer_step_(qg, kk, vv, qw, kw, KC, VC, position=cap - 1,
                                               positions=positions, sections=sections,
                                               frequency_base=1e7, epsilon=1e-6)
            return (out,)

        def refresh(rng):
            for x, s in ((qg, 3.0), (kk, 3.0), (vv, 1.0)):
                x.copy_(rnd(x.shape, s))
            positions.copy_(torch.from_numpy(rng.integers(0, cap, B).astype(np.int32)).to(gpu))
        return step, refresh, [KC, VC]
    # recurrent_layer_step (fp32 end to end)
    hk, hv, dk, dv, kernel = hkv, hkv * min(c["group"], 2), d, 64, 4
    chn = 2 * hk * dk + hv * dv
    ws = ops.initialize_recurrent_workspace(batch_size=B, convolution_kernel=kernel,
                                            convolution_channels=chn, value_heads=hv,
                                            value_dimension=dv, key_dimension=dk)
    ws.delta_state.copy_(torch.randn(ws.delta_state.shape, generator=g, device=gpu) * 0.1)
    ws.convolution_history.copy_(torch.randn(ws.convolution_history.shape, generator=g,
                                             device=gpu))
    mixed, gate = rnd((B, chn)), rnd((B, hv * dv))
    bl, al = rnd((B, hv)), rnd((B, hv))
    w = rnd((kernel, chn), 0.5)
    dt = rnd((hv,))
    ssm = -torch.exp(torch.rand(hv, generator=g, device=gpu) * 2 - 1)
    nw = torch.rand(dv, generator=g, device=gpu) + 0.5
    inputs = [mixed, gate, bl, al]

    def step():
        return (ops.recurrent_layer_step_(ws, mixed, w, gate, bl, al, dt, ssm, nw, key_heads=hk,
                                          key_dimension=dk, epsilon=1e-6),)

    def refresh(rng):
        for x in inputs:
            x.copy_(rnd(x.shape))
    return step, refresh, [ws.delta_state, ws.convolution_history]


def _bits(t):
    import torch
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


@pytest.mark.parametrize("c", CASES, ids=[c["id"] for c in CASES])
def test_captured_call_replays_equal_eager(gpu, ops, c):
    import torch
    print("graph replay:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    step, refresh, states = _setup(torch, ops, gpu, c)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs_g = step()
    torch.cuda.synchronize()
    for i in range(3):
        refresh(rng)
        saved = [s.clone() for s in states]
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs_g] + [s.clone() for s in states]
        for s, v in zip(states, saved):
            s.copy_(v)
        want = list(step()) + [s.clone() for s in states]
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(_bits(a), _bits(b)), (c["id"], i, j)
