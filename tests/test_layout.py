"""Fragment-tiled expert weight layout (host side, CPU): the permutation that
tile_weights applies is checked element by element against the layout
definition in include/dsk.h (DSK_LAYOUT_TILED), and untile_weights inverts it."""
import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def dsk():
    import ds_kernels
    return ds_kernels


@pytest.mark.parametrize("G,N,K", [(1, 32, 16), (2, 64, 48), (3, 96, 128)])
def test_tile_matches_layout_definition(dsk, G, N, K):
    w = torch.arange(G * N * K, dtype=torch.int64).reshape(G, N, K)
    t = dsk.tile_weights(w)
    assert tuple(t.shape) == (G, N // 32, K // 16, 64, 8)
    flat = t.reshape(G, -1).numpy()
    wn = w.numpy()
    for g in range(G):
        for n in range(N):
            for k in range(K):
                rb, r, ks, kk = n // 32, n % 32, k // 16, k % 16
                pos = (rb * (K // 16) + ks) * 512 + ((kk // 8) * 32 + r) * 8 + kk % 8
                assert flat[g, pos] == wn[g, n, k]


def test_untile_inverts_tile(dsk):
    w = torch.randn(2, 64, 64).to(torch.bfloat16)
    assert torch.equal(dsk.untile_weights(dsk.tile_weights(w)), w)


def test_tile_rejects_ragged_shapes(dsk):
    with pytest.raises(ValueError):
        dsk.tile_weights(torch.zeros(1, 48, 16))
    with pytest.raises(ValueError):
        dsk.tile_weights(torch.zeros(1, 32, 24))


def test_fragment_lane_order(dsk):
    """Lane l of a fragment holds row l % 32, columns 8*(l // 32) .. +7: the
    operand order of v_mfma_f32_32x32x16_bf16."""
    w = torch.arange(32 * 16, dtype=torch.int64).reshape(1, 32, 16)
    frag = dsk.tile_weights(w)[0, 0, 0].numpy()  # [64, 8]
    for lane in range(64):
        np.testing.assert_array_equal(
            frag[lane], w[0, lane % 32, 8 * (lane // 32):8 * (lane // 32) + 8].numpy())


@pytest.mark.parametrize("tiled", [True, False])
def test_mla_merged_projection_weight_views(dsk, tiled):
    """MLAWeights keeps q_proj and kv_a_proj in one [q rows; kva rows] matrix for
    the single prefill GEMM; its q and kva fields are leading-dim slices of it and
    equal the separately packed weights (tiled: 32-row blocks stay in order)."""
    from ds_kernels import mla as dm
    g = torch.Generator().manual_seed(4)
    w = {"q": torch.randn(3072, 256, generator=g), "kva": torch.randn(576, 256, generator=g),
         "kva_norm": torch.ones(512), "kvb": torch.randn(4096, 512, generator=g),
         "o": torch.randn(256, 2048, generator=g)}
    W = dm.MLAWeights.from_tensors(w, torch.device("cpu"), tiled=tiled)
    pack = (lambda t: dsk.tile_weights(t.to(torch.bfloat16)[None])[0]) if tiled else \
        (lambda t: t.to(torch.bfloat16))
    assert torch.equal(W.q, pack(w["q"])) and torch.equal(W.kva, pack(w["kva"]))
    assert W.q.data_ptr() == W.q_kva.data_ptr()
    assert W.q.is_contiguous() and W.kva.is_contiguous()
