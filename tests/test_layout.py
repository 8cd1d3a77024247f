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
