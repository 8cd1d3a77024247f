"""LatentKVCache API (the buffer bookkeeping of src/kernels/mla_cache.py:29-219)
on CPU tensors: shapes, views, append/read-back, overflow and argument errors,
memory accounting and repr. The reference ships no tests for this class; the
expected values follow from its documented contract (mla_cache.py:1-23: 576
bf16 values per token, 4.5 MB per layer at bsz=1, max_seq=4096)."""
import pytest
import torch

from ds_kernels import LatentKVCache


def _tokens(b, n, seed, width):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(b, n, width, generator=g).to(torch.bfloat16)


def test_shapes_and_memory_of_the_inference_cache():
    c = LatentKVCache.for_inference(1, device="cpu")
    assert c.kv_latent.shape == (1, 4096, 512) and c.k_pe_cache.shape == (1, 4096, 64)
    assert c.kv_latent.dtype == torch.bfloat16
    assert c.memory_bytes == 576 * 4096 * 2 == int(4.5 * 1024 ** 2)
    assert c.current_len == 0 and c.remaining_capacity == 4096
    assert repr(c) == ("LatentKVCache(bsz=1, tokens=0/4096, used=0.00MB/4.50MB, device=cpu, "
                       "dtype=torch.bfloat16)")


def test_update_get_round_trip_and_views():
    c = LatentKVCache(2, 10, device="cpu")
    lat1, pe1 = _tokens(2, 3, 0, 512), _tokens(2, 3, 1, 64)
    lat2, pe2 = _tokens(2, 4, 2, 512), _tokens(2, 4, 3, 64)
    c.update(lat1, pe1)
    c.update(lat2, pe2)
    assert c.current_len == 7 and c.remaining_capacity == 3
    lat, pe = c.get()
    assert torch.equal(lat, torch.cat([lat1, lat2], 1)) and torch.equal(pe, torch.cat([pe1, pe2], 1))
    lat, pe = c.get(3)
    assert torch.equal(lat, lat1) and torch.equal(pe, pe1)
    # zero-copy views of the cache buffers
    assert lat.data_ptr() == c.kv_latent.data_ptr() and pe.data_ptr() == c.k_pe_cache.data_ptr()
    # one row per token: latent then RoPE key, as kv_a_proj_with_mqa emits them,
    # then the rotated key (written by the first attention over the token)
    assert c.rows.shape == (2, 10, 640)
    assert torch.equal(c.rows[:, :7, :512], c.get()[0])
    assert torch.equal(c.rows[:, 3:7, 512:576], pe2)
    assert c.k_rope.shape == (2, 10, 64) and c.k_rope.data_ptr() == c.rows[..., 576:].data_ptr()
    assert c.get(0)[0].shape == (2, 0, 512)


def test_update_converts_dtype():
    c = LatentKVCache(1, 4, device="cpu")
    lat = torch.randn(1, 2, 512)
    c.update(lat, torch.randn(1, 2, 64))
    assert torch.equal(c.get()[0], lat.to(torch.bfloat16))


def test_overflow_raises_and_writes_nothing():
    c = LatentKVCache(1, 5, device="cpu")
    c.update(_tokens(1, 4, 0, 512), _tokens(1, 4, 1, 64))
    before = c.rows.clone()
    with pytest.raises(RuntimeError, match="KV cache overflow: current_len=4, new_tokens=2, max_seq=5"):
        c.update(_tokens(1, 2, 2, 512), _tokens(1, 2, 3, 64))
    assert c.current_len == 4 and torch.equal(c.rows, before)
    c.update(_tokens(1, 1, 4, 512), _tokens(1, 1, 5, 64))
    assert c.current_len == 5 and c.remaining_capacity == 0


def test_argument_errors():
    with pytest.raises(ValueError, match="bsz"):
        LatentKVCache(0, 4, device="cpu")
    with pytest.raises(ValueError, match="max_seq"):
        LatentKVCache(1, 2.5, device="cpu")
    c = LatentKVCache(1, 4, device="cpu")
    with pytest.raises(ValueError, match="compressed_kv must be 3D"):
        c.update(torch.zeros(2, 512), torch.zeros(1, 2, 64))
    with pytest.raises(ValueError, match="k_pe must be 3D"):
        c.update(torch.zeros(1, 2, 512), torch.zeros(2, 64))
    with pytest.raises(ValueError, match="seq_len=1"):
        c.get(1)


def test_reset_keeps_buffers_and_repr_counts_used_tokens():
    c = LatentKVCache(2, 1024, device="cpu")
    ptr = c.rows.data_ptr()
    c.update(_tokens(2, 512, 0, 512), _tokens(2, 512, 1, 64))
    # used = 512 tokens * 576 * 2 B * bsz 2 = 1.125 MiB of 2.25 MiB
    assert "tokens=512/1024, used=1.12MB/2.25MB" in repr(c)
    c.reset()
    assert c.current_len == 0 and c.remaining_capacity == 1024 and c.rows.data_ptr() == ptr


def test_append_slots_reserves_views_in_order():
    c = LatentKVCache(2, 6, device="cpu")
    c.update(_tokens(2, 2, 0, 512), _tokens(2, 2, 1, 64))
    rows = c.append_slots(3)
    assert rows.shape == (2, 3, 576) and c.current_len == 5
    rows.copy_(_tokens(2, 3, 2, 576))
    lat, pe = c.get()
    assert torch.equal(lat[:, 2:], rows[..., :512]) and torch.equal(pe[:, 2:], rows[..., 512:])
    assert rows.data_ptr() == c.rows[:, 2:].data_ptr()
    with pytest.raises(RuntimeError, match="KV cache overflow: current_len=5, new_tokens=2"):
        c.append_slots(2)
    assert c.current_len == 5


def test_rotated_key_count_follows_the_rows():
    """rope_len counts the leading positions whose rotated key is valid: rows
    rewritten by update / append_slots (after a rollback of the length, or a
    reset) drop out of it."""
    c = LatentKVCache(1, 8, device="cpu")
    c.update(_tokens(1, 4, 0, 512), _tokens(1, 4, 1, 64))
    assert c.rope_len == 0
    c._rope_len = 4                      # as an attention over the 4 tokens leaves it
    assert c.rope_len == 4
    c.append_slots(2)
    assert c.rope_len == 4 and c.current_len == 6
    c._len = 3                           # roll back: row 3 will be rewritten
    c.update(_tokens(1, 1, 2, 512), _tokens(1, 1, 3, 64))
    assert c.rope_len == 3 and c.current_len == 4
    c.reset()
    assert c.rope_len == 0


def test_rejected_decode_step_leaves_the_cache_length():
    """mla_decode_forward checks its inputs before it reserves cache slots, and
    gives the slots back if a later step raises: a caller that catches the error
    and carries on never attends over rows that were not written. The reference
    update() advances the length only after its writes (mla_cache.py:131-143)."""
    from ds_kernels import mla_decode_forward
    from ds_kernels import mla as dm
    from ds_kernels import synthetic as syn
    W = dm.MLAWeights.from_tensors(syn.mla_weights(), torch.device("cpu"))
    c = LatentKVCache(1, 16, device="cpu")
    c.update(_tokens(1, 5, 0, 512), _tokens(1, 5, 1, 64))
    cos, sin = dm.yarn_cos_sin(16)
    cos, sin = cos.to(torch.bfloat16), sin.to(torch.bfloat16)
    x = _tokens(1, 2, 2, 2048)
    with pytest.raises(RuntimeError, match="cos must be"):           # table too short
        mla_decode_forward(x, W, c, cos[:6], sin[:6])
    with pytest.raises(RuntimeError, match="hidden size 1024"):
        mla_decode_forward(_tokens(1, 2, 3, 1024), W, c, cos, sin)
    c32, s32 = (t.to(torch.bfloat16) for t in dm.yarn_cos_sin(32))
    with pytest.raises(RuntimeError, match="KV cache overflow"):
        mla_decode_forward(_tokens(1, 12, 4, 2048), W, c, c32, s32)
    assert c.current_len == 5
    # valid shapes, but the tensors are on the CPU: the projection rejects them
    # after the slots were reserved, and the reservation is undone
    with pytest.raises(RuntimeError, match="CUDA"):
        mla_decode_forward(x, W, c, cos, sin)
    assert c.current_len == 5


def test_rope_tables_identity_and_reset_rope():
    """Rotated keys belong to the tables that made them: other tables (or the
    same tensor modified in place) drop them, reset_rope() drops them after
    direct writes into the planes."""
    c = LatentKVCache(1, 8, kv_lora_rank=16, rope_head_dim=8, device="cpu")
    c.update(torch.zeros(1, 4, 16), torch.zeros(1, 4, 8))
    cos, sin = torch.ones(8, 8), torch.zeros(8, 8)
    c.use_rope_tables(cos, sin)
    c._rope_len = 4                      # as a decode step leaves it
    c.use_rope_tables(cos, sin)          # same tables: kept
    assert c.rope_len == 4
    c.use_rope_tables(cos.clone(), sin)  # another tensor: dropped
    assert c.rope_len == 0
    c._rope_len = 4
    c.use_rope_tables(cos, sin)          # back to the first tensor: also new
    assert c.rope_len == 0
    c._rope_len = 4
    cos.mul_(2)                          # modified in place
    c.use_rope_tables(cos, sin)
    assert c.rope_len == 0
    c._rope_len = 4
    c.k_pe_cache[:, :2] = 1.0            # direct write into the raw keys
    c.reset_rope()
    assert c.rope_len == 0 and c.current_len == 4


def test_rope_tables_growing_views_and_recycled_memory():
    """Views of one table with a growing position count (cos[:seq_len], as the
    reference's rotary embedding returns them each step) keep the rotated keys;
    a table freed and replaced by new values cannot alias the old one, because
    the cache holds the tables it used."""
    c = LatentKVCache(1, 8, kv_lora_rank=16, rope_head_dim=8, device="cpu")
    c.update(torch.zeros(1, 4, 16), torch.zeros(1, 4, 8))
    cos_full, sin_full = torch.rand(16, 8), torch.rand(16, 8)
    c.use_rope_tables(cos_full[:4], sin_full[:4])
    c._rope_len = 4
    c.use_rope_tables(cos_full[:5], sin_full[:5])   # same rows, one more position
    assert c.rope_len == 4
    c.use_rope_tables(cos_full[1:6], sin_full[1:6])  # shifted rows: other positions
    assert c.rope_len == 0
    # per-sequence tables [b, s, d]: the batch dims count, the length does not
    cb = torch.rand(2, 16, 8)
    c.use_rope_tables(cb[:, :4], cb[:, :4])
    c._rope_len = 4
    c.use_rope_tables(cb[:, :6], cb[:, :6])
    assert c.rope_len == 4
    c.use_rope_tables(cb[:1, :6], cb[:1, :6])
    assert c.rope_len == 0
    # the tables in use stay alive: a new tensor never takes their address
    c._rope_len = 4
    held = c._rope_tables[1].data_ptr()
    del cb
    fresh = [torch.rand(1, 6, 8) for _ in range(8)]
    assert all(t.data_ptr() != held for t in fresh)
    c.use_rope_tables(fresh[0], fresh[0])
    assert c.rope_len == 0
