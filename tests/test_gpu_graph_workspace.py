"""GPU regression: a captured graph keeps the workspace it was captured with.

The facades share one grow-only scratch workspace per device.  A HIP graph
that captures a decode call holds that workspace's address in its kernel
arguments; when a later call needs more room the module allocates a larger
workspace, and the old one must stay allocated, or the graph's replays
would write split partials into memory torch has since given to other
tensors.  The test captures a decode, forces the workspace to grow, fills
the caching allocator with sentinel tensors, replays, and checks that the
replays equal the eager call bit for bit and that no sentinel changed.
"""

import importlib

import pytest

pytestmark = pytest.mark.gpu


def _mod(name):
    return importlib.import_module("alpacca-open-sourced-by-jt_amd." + name)


def test_graph_replay_after_workspace_growth(gpu):
    import torch
    lib = _mod("_lib")
    ops_c = _mod("_ops")
    g = torch.Generator(device=gpu).manual_seed(7)
    bf = torch.bfloat16
    b, hq, hkv, d, cap = 2, 8, 2, 128, 1024
    K = torch.randn((cap, b, hkv, d), generator=g, device=gpu).to(bf)
    V = torch.randn((cap, b, hkv, d), generator=g, device=gpu).to(bf)
    q = torch.zeros((b, hq, d), dtype=bf, device=gpu)
    strides = (hkv * b * d, hkv * d, d)

    def step():
        return ops_c.decode(q, K, V, length=cap, k_strides=strides, v_strides=strides,
                            batch=b, kv_heads=hkv)

    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream(gpu).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = step()
    torch.cuda.synchronize()

    held = lib._workspaces[str(gpu)]
    held_ptr, held_bytes = held.data_ptr(), held.numel()
    del held
    grown = lib.workspace(torch, gpu, 2 * held_bytes + (1 << 20))
    assert grown.data_ptr() != held_ptr
    # sentinels of the retired workspace's size: the caching allocator would
    # hand its block to one of these had it been released
    sentinels = [torch.full((held_bytes,), 0x5A, dtype=torch.uint8, device=gpu)
                 for _ in range(4)]
    for i in range(4):
        q.copy_(torch.randn(q.shape, generator=g, device=gpu).to(bf))
        graph.replay()
        torch.cuda.synchronize()
        out_e = step()  # eager: runs on the grown workspace
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16)), i
    for s in sentinels:
        assert bool((s == 0x5A).all())
