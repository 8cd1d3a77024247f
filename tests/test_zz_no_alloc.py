"""The allocation-free layer entry (dsk_moe_layer_forward_noalloc), called
through the C ABI, against dsk_moe_layer_forward with a caller workspace: the
same kernels on the same inputs, so outputs, routing indices and weights and
expert offsets must agree bit for bit. Two calls in a row on one GPU, the
second with fewer tokens, show that nothing left in the shared static scratch
by the first call leaks into the second; a layer larger than the scratch is
rejected with a status and a message."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
E, K, H, I = 64, 6, 2048, 1408


@pytest.fixture(scope="module")
def dsk():
    import ds_kernels
    return ds_kernels


@pytest.fixture(scope="module")
def layer(dsk):
    from ds_kernels import synthetic as syn
    W = syn.moe_weights()
    w1, w2, nsh = dsk.pack_tensors(W.gates, W.ups, W.downs, device=DEV, shared=W.shared)
    wg = W.wg.to(torch.bfloat16)
    tiled = (dsk.tile_weights(w1), dsk.tile_weights(w2),
             dsk.tile_weights(wg[None])[0].to(DEV))
    row_major = (w1, w2, wg.to(DEV))
    return {"tiled": tiled, "row_major": row_major, "nsh": nsh,
            "bias": syn.zipf_router_bias().to(DEV)}


def _noalloc(dsk, x, wg, bias, w1, w2, nsh, tiled, expect_rc=0):
    T = x.shape[0]
    out = torch.empty((T, H), dtype=torch.bfloat16, device=DEV)
    idx = torch.empty((T, K), dtype=torch.int32, device=DEV)
    w = torch.empty((T, K), dtype=torch.float32, device=DEV)
    offs = torch.empty((E + 1,), dtype=torch.int32, device=DEV)
    with torch.cuda.device(DEV):
        rc = dsk.lib.dsk_moe_layer_forward_noalloc(
            x.data_ptr(), wg.data_ptr(), bias.data_ptr() if bias is not None else None,
            w1.data_ptr(), w2.data_ptr(), out.data_ptr(), T, E, K, nsh, H, I,
            1 if tiled else 0, idx.data_ptr(), w.data_ptr(), offs.data_ptr(), None,
            torch.cuda.current_stream(DEV).cuda_stream)
    if expect_rc != 0:
        assert rc == expect_rc, rc
        return dsk.lib.dsk_last_error().decode()
    assert rc == 0, dsk.lib.dsk_last_error().decode()
    return out, idx, w, offs


@pytest.mark.parametrize("layout,sizes", [("tiled", (64, 16)), ("tiled", (128, 1)),
                                          ("row_major", (16, 4))])
def test_noalloc_matches_workspace_entry(dsk, layer, layout, sizes):
    from ds_kernels import synthetic as syn
    w1, w2, wg = layer[layout]
    nsh, bias = layer["nsh"], layer["bias"]
    for T in sizes:
        print(f"noalloc layout={layout} T={T}", flush=True)
        x = syn.tokens(T, seed=1000 + T).to(torch.bfloat16).to(DEV)
        got, gidx, gw, goffs = _noalloc(dsk, x, wg, bias, w1, w2, nsh, layout == "tiled")
        ref, (ridx, rw, roffs) = dsk.moe_layer_forward(x, wg, w1, w2, K, nsh, gate_bias=bias,
                                                      return_routing=True)
        torch.cuda.synchronize()
        assert torch.equal(gidx, ridx)
        assert torch.equal(gw, rw)
        assert torch.equal(goffs, roffs)
        assert torch.equal(got, ref), f"T={T}: outputs differ"
        assert bool(torch.isfinite(got.float()).all())


def test_noalloc_rejects_layers_beyond_the_scratch(dsk, layer):
    """T=4096 needs ~240 MB of scratch: rejected before any launch, with a
    message naming the limit; the same call at T=128 is accepted."""
    lib = dsk.lib
    need = lib.dsk_moe_layer_workspace_size(4096, E, K, 2, H, I)
    assert need > 8 << 20
    assert lib.dsk_moe_layer_workspace_size(128, E, K, 2, H, I) <= 8 << 20
    w1, w2, wg = layer["tiled"]
    x = torch.zeros((4096, H), dtype=torch.bfloat16, device=DEV)
    out = torch.full((4096, H), 7, dtype=torch.bfloat16, device=DEV)
    rc = lib.dsk_moe_layer_forward_noalloc(
        x.data_ptr(), wg.data_ptr(), None, w1.data_ptr(), w2.data_ptr(), out.data_ptr(),
        4096, E, K, 2, H, I, 1, None, None, None, None,
        torch.cuda.current_stream(DEV).cuda_stream)
    msg = lib.dsk_last_error().decode()
    assert rc == 5 and "scratch" in msg and str(need) in msg, (rc, msg)
    torch.cuda.synchronize()
    assert bool((out == 7).all()), "a rejected call must not write its output"


def _busy(stream):
    """Keep `stream` busy for a while (bounded work): a chain of matrix products."""
    with torch.cuda.stream(stream):
        a = torch.randn(4096, 4096, device=DEV)
        for _ in range(24):
            a = torch.mm(a, a) * 1e-3


def test_noalloc_refuses_overlap_on_another_stream(dsk, layer):
    """Two calls that would share the static scratch at the same time: while a
    call is in flight on one stream, a call on another stream of the GPU is
    refused with a status and a message (not run over the first one's data);
    once the first has finished, the second stream is accepted and its result
    equals the workspace entry's."""
    from ds_kernels import synthetic as syn
    w1, w2, wg = layer["tiled"]
    nsh, bias = layer["nsh"], layer["bias"]
    x = syn.tokens(16, seed=3).to(torch.bfloat16).to(DEV)
    s1, s2 = torch.cuda.Stream(DEV), torch.cuda.Stream(DEV)
    torch.cuda.synchronize()
    _busy(s1)
    with torch.cuda.stream(s1):
        _noalloc(dsk, x, wg, bias, w1, w2, nsh, True)
    with torch.cuda.stream(s2):
        msg = _noalloc(dsk, x, wg, bias, w1, w2, nsh, True, expect_rc=1)
    assert "another stream" in msg, msg
    torch.cuda.synchronize()
    with torch.cuda.stream(s2):
        got, *_ = _noalloc(dsk, x, wg, bias, w1, w2, nsh, True)
    ref = dsk.moe_layer_forward(x, wg, w1, w2, K, nsh, gate_bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("T", [1, 16])
def test_noalloc_under_graph_capture(dsk, layer, T):
    """After an eager call on the device, the entry can be captured into a HIP
    graph; every replay (with eager calls on other inputs in between) gives the
    eager result bit for bit."""
    from ds_kernels import synthetic as syn
    w1, w2, wg = layer["tiled"]
    nsh, bias = layer["nsh"], layer["bias"]
    x = syn.tokens(T, seed=50 + T).to(torch.bfloat16).to(DEV)
    x_other = syn.tokens(T + 3, seed=60 + T).to(torch.bfloat16).to(DEV)
    ref, ridx, rw, roffs = _noalloc(dsk, x, wg, bias, w1, w2, nsh, True)
    torch.cuda.synchronize()
    ref = ref.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(DEV)
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out, idx, w, offs = _noalloc(dsk, x, wg, bias, w1, w2, nsh, True)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        _noalloc(dsk, x_other, wg, bias, w1, w2, nsh, True)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(idx, ridx) and torch.equal(offs, roffs)
    del g
