"""C-ABI checks that need no GPU: libdsk.so loads, exports every function
declared in include/dsk.h, and rejects bad arguments with a status code and a
message before touching the device (reference error behaviour: TORCH_CHECK /
std::runtime_error -> RuntimeError)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsk.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(dsk_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def dsk():
    import ds_kernels
    return ds_kernels


def test_every_declared_symbol_is_exported(dsk):
    names = declared_functions()
    assert len(names) >= 20
    raw = ctypes.CDLL(dsk.LIB_PATH)
    missing = [n for n in names if not hasattr(raw, n)]
    assert not missing, f"not exported: {missing}"
    from ds_kernels._lib import SIGNATURES
    assert set(names) == set(SIGNATURES), "python binding out of sync with include/dsk.h"


def test_abi_version(dsk):
    assert dsk.lib.dsk_abi_version() == 3


def _err(dsk):
    return dsk.lib.dsk_last_error().decode()


def test_error_text_is_per_thread(dsk):
    """dsk_last_error() is thread-local: two threads failing different checks at the
    same time each read their own message (ctypes releases the GIL around calls)."""
    import threading
    lib = dsk.lib
    seen = {0: set(), 1: set()}

    def worker(i):
        for _ in range(300):
            if i == 0:
                rc = lib.dsk_moe_routing(None, 65, None, None, 8, 4, 65, 6, None, 0, None)
            else:
                rc = lib.dsk_moe_routing(None, 64, None, None, 8, 4, 64, 7, None, 0, None)
            seen[i].add((rc, lib.dsk_last_error().decode()))

    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert len(seen[0]) == 1 and len(seen[1]) == 1
    (rc0, m0), = seen[0]
    (rc1, m1), = seen[1]
    assert rc0 == rc1 == 1 and "num_experts" in m0 and "top_k" in m1


def test_linear_split_validation(dsk):
    lib = dsk.lib
    # argument order: x, ld_x, w, out0, ld_out0, out1, ld_out1, M, K, N, n_split, stream
    def call(n_split=3072, ld0=3072, ld1=576, out1=16, M=1, N=3648):
        return lib.dsk_linear_split(16, 2048, 16, 16, ld0, out1, ld1, M, 2048, N, n_split, None)
    assert call(n_split=3000) == 1 and "multiple of 64" in _err(dsk)
    assert call(n_split=3648) == 1 and "multiple of 64" in _err(dsk)
    assert call(ld0=3000) == 1 and "ld_out0" in _err(dsk)
    assert call(ld1=500) == 1 and "ld_out1" in _err(dsk)
    assert call(out1=None) == 2
    assert call(out1=20) == 3 and "8-byte" in _err(dsk)
    assert call(M=0) == 0  # nothing to do, nothing launched


def test_routing_limits_rejected(dsk):
    lib = dsk.lib
    rc = lib.dsk_moe_routing(None, 65, None, None, 8, 4, 65, 6, None, 0, None)
    assert rc == 1 and "num_experts" in _err(dsk)
    rc = lib.dsk_moe_routing(None, 64, None, None, 8, 4, 64, 7, None, 0, None)
    assert rc == 1 and "top_k" in _err(dsk)
    rc = lib.dsk_moe_routing(None, 64, None, None, None, 4, 64, 6, None, 0, None)
    assert rc == 2


def test_dispatch_and_combine_validation(dsk):
    lib = dsk.lib
    rc = lib.dsk_moe_dispatch(None, 2044, None, None, None, None, None, None, 4, 2044, 64, 6,
                              None, 0, None)
    assert rc == 1 and "divisible by 8" in _err(dsk)
    rc = lib.dsk_moe_combine(None, None, None, None, 6, 0, 2048, None, 0, None)
    assert rc == 1 and "num_tokens must be positive" in _err(dsk)


def test_gemm_validation(dsk):
    lib = dsk.lib
    # K not a multiple of 64
    rc = lib.dsk_moe_gemm1(16, 16, 16, 16, 6, 64, 100, 2816, None)
    assert rc == 1 and "multiple of 64" in _err(dsk)
    # misaligned pointers
    rc = lib.dsk_moe_gemm2(18, 16, 16, 16, 6, 64, 1408, 2048, None)
    assert rc == 3
    # too many groups
    rc = lib.dsk_moe_gemm2(16, 16, 16, 16, 6, 200, 1408, 2048, None)
    assert rc == 1


def test_linear_ex_validation(dsk):
    lib = dsk.lib
    # unknown weight layout
    rc = lib.dsk_linear_ex(16, 2048, 16, 7, 16, 576, 4, 2048, 576, None)
    assert rc == 1 and "layout" in _err(dsk)
    # tiled weights need N % 32 == 0
    rc = lib.dsk_linear_ex(16, 2048, 16, 1, 16, 100, 4, 2048, 100, None)
    assert rc == 1 and "32" in _err(dsk)
    # K must be a multiple of 64
    rc = lib.dsk_linear_ex(16, 96, 16, 1, 16, 64, 4, 96, 64, None)
    assert rc == 1 and "multiple of 64" in _err(dsk)


def test_attn_softmax_validation(dsk):
    lib = dsk.lib
    # rows padded to 8 keys: ld must cover kv_len rounded up to 8 and be a multiple of 8
    rc = lib.dsk_attn_softmax(16, 100, 64, 100, 8, 0.1, 1, None)
    assert rc == 3 and "rounded up to 8" in _err(dsk)
    rc = lib.dsk_attn_softmax(16, 104, 64, 105, 8, 0.1, 1, None)
    assert rc == 3 and "rounded up to 8" in _err(dsk)
    rc = lib.dsk_attn_softmax(None, 104, 64, 100, 8, 0.1, 1, None)
    assert rc == 2       # a valid padded shape gets past the size checks
    rc = lib.dsk_attn_softmax(None, 8192, 64, 8192, 8, 0.1, 1, None)
    assert rc == 2       # rows longer than 4096 keys are accepted (two-pass kernel)
    rc = lib.dsk_attn_softmax(16, 64, 60, 64, 8, 0.1, 1, None)
    assert rc == 1 and "q_len" in _err(dsk)
    rc = lib.dsk_attn_softmax(16, 64, 64, 64, 128, 0.1, 1, None)
    assert rc == 1 and "q_len" in _err(dsk)


def test_attn_softmax_masked_validation(dsk):
    lib = dsk.lib
    # mask dtype must be bf16 (0) or fp32 (1)
    rc = lib.dsk_attn_softmax_masked(16, 64, 64, 64, 8, 1, 0.1, 0, 16, 7, 0, 0, 64, None)
    assert rc == 1 and "mask dtype" in _err(dsk)
    # rows / q_len must be a multiple of heads
    rc = lib.dsk_attn_softmax_masked(16, 64, 64, 64, 8, 3, 0.1, 0, 16, 1, 0, 0, 64, None)
    assert rc == 1 and "heads" in _err(dsk)
    rc = lib.dsk_attn_softmax_masked(16, 64, 64, 64, 8, 2, 0.1, 0, None, 1, 0, 0, 64, None)
    assert rc == 2 and "mask" in _err(dsk)
    assert lib.dsk_attn_softmax_masked(None, 64, 0, 64, 8, 2, 0.1, 0, None, 1, 0, 0, 64,
                                       None) == 0


def test_linear_rows_validation(dsk):
    lib = dsk.lib

    def call(M=1, K=2048, N=2048, n_split=2048, x=16, ld_x=2048, out0=16, out1=None, batch=1):
        return lib.dsk_linear_rows(x, ld_x, 0, 16, 0, out0, 2048, 0, out1, 0, 0, n_split, batch,
                                   M, K, N, None)
    assert call(M=0) == 0 and call(batch=0, x=None) == 0
    assert call(M=5) == 1 and "4 token rows" in _err(dsk)
    assert call(K=2000) == 1 and "multiple of 128" in _err(dsk)
    assert call(N=2040, n_split=2040) == 1 and "multiple of 128" in _err(dsk)
    assert call(n_split=2049) == 1 and "n_split" in _err(dsk)
    assert call(n_split=1024) == 2 and "NULL" in _err(dsk)
    assert call(x=None) == 2
    assert call(x=24) == 3 and call(ld_x=2052) == 3
    assert call(ld_x=1024, K=2048) == 1 and "row stride" in _err(dsk)


def test_attn_pack_validation(dsk):
    lib = dsk.lib

    def call(q=16, ld_q=3648, kv=16, ld_kv=4096, kpe=16, ld_kpe=3648, ld_cs=64, out=16,
             batch=2, seq=64, heads=16, dims=(128, 64, 128)):
        return lib.dsk_mla_attn_pack(q, ld_q, kv, ld_kv, kpe, ld_kpe, 16, 16, ld_cs, out, 16, 16,
                                     batch, seq, heads, dims[0], dims[1], dims[2], None)
    assert call(seq=0) == 0 and call(batch=0, q=None) == 0
    assert call(dims=(128, 32, 128)) == 1 and "head dims" in _err(dsk)
    assert call(seq=60) == 1 and "multiple of 8" in _err(dsk)
    assert call(heads=70000) == 1 and "65535" in _err(dsk)
    assert call(q=None) == 2 and "NULL" in _err(dsk)
    assert call(out=24) == 3 and call(ld_kpe=3650) == 3
    assert call(ld_q=3064) == 1 and "row stride" in _err(dsk)
    assert call(ld_kv=4088) == 1 and call(ld_cs=56) == 1


def test_attn_pack_ex_validation(dsk):
    lib = dsk.lib

    def call(seq=60, seq_pad=64, cs_bs=0, q=16):
        return lib.dsk_mla_attn_pack_ex(q, 3648, 16, 4096, 16, 3648, 16, 16, 64, cs_bs, 16, 16,
                                        16, 2, seq, seq_pad, 16, 128, 64, 128, None)
    assert call(q=None) == 2                    # seq 60 padded to 64 passes the size checks
    assert call(seq_pad=60) == 1 and "seq_pad" in _err(dsk)
    assert call(seq_pad=72) == 1 and "seq_pad" in _err(dsk)
    assert call(cs_bs=4) == 3                   # per-batch tables must start 16-byte aligned
    assert call(cs_bs=-64) == 1 and "stride" in _err(dsk)


def test_mla_decode_split_plan(dsk):
    """Key splits per query token, read back from the workspace size (a 32 KB
    partial and 128 B of running max and sum per split and token): about 256
    workgroups; a plan of one 64-key block per split takes two where that
    leaves 128 or more workgroups; plans of several blocks are left alone."""
    per_split = (16 * 512 + 32) * 4

    def splits(b, n, L):
        ws = dsk.lib.dsk_mla_decode_workspace_size(b, n, L)
        return ws // (b * n * per_split)
    assert splits(1, 1, 4096) == 64     # one block each: only 64 workgroups
    assert splits(3, 1, 4096) == 64     # two blocks would leave 96 workgroups
    assert splits(4, 1, 4096) == 32     # two blocks each: 128 workgroups
    assert splits(8, 1, 4096) == 32
    assert splits(16, 1, 4096) == 16    # four blocks each
    assert splits(1, 8, 4096) == 32
    assert splits(2, 4, 4096) == 32
    assert splits(8, 1, 2100) == 17     # 33 blocks: two per split, not three
    assert splits(4, 1, 2100) == 33     # two per split would leave 68 workgroups
    assert splits(64, 1, 4096) == 4


def test_mla_decode_validation(dsk):
    lib = dsk.lib
    ws = lib.dsk_mla_decode_workspace_size(1, 1, 4096)
    assert ws == 64 * (16 * 512 + 32) * 4
    assert lib.dsk_mla_decode_workspace_size(2, 3, 65) == 2 * 3 * 2 * (16 * 512 + 32) * 4
    assert lib.dsk_mla_decode_workspace_size(1, 600, 4096) == 256  # one split per token: no partials
    # argument order: q_abs, qa_tok, qa_head, q_pe, qp_tok, qp_head, latent, k_pe, k_rope,
    # rope_len, ld_tok, ld_batch, cos, sin, eps, scale, batch, q_len, kv_len, out, o_tok,
    # o_head, ws, bytes, stream
    # one 640-wide cache row per token: latent at column 0, k_pe at 512, k_rope at 576
    lat, kpe, krope = 1 << 20, (1 << 20) + 1024, (1 << 20) + 1152

    def call(q_len=1, kv_len=64, ld_tok=640, ld_batch=640 * 64, batch=1, qa=(8192, 512),
             out=16, bytes_=1 << 30, q_abs=16, k_rope=krope, rope_len=0):
        return lib.dsk_mla_decode_attention(q_abs, qa[0], qa[1], 16, 3072, 192, lat, kpe, k_rope,
                                            rope_len, ld_tok, ld_batch, 16, 16, 1e-6, 0.1, batch,
                                            q_len, kv_len, out, 8192, 512, 16, bytes_, None)
    assert lib.dsk_mla_decode_attention(None, 0, 0, None, 0, 0, None, None, None, 0, 0, 0, None,
                                        None, 1e-6, 0.1, 0, 1, 64, None, 0, 0, None, 0, None) == 0
    assert call(rope_len=65) == 1 and "rope_len" in _err(dsk)
    assert call(rope_len=-1) == 1 and "rope_len" in _err(dsk)
    assert call(k_rope=None) == 2
    assert call(k_rope=24) == 3
    assert call(kv_len=1 << 21, ld_batch=640 << 21) == 1 and "2 GiB" in _err(dsk)
    assert call(q_len=65) == 1 and "q_len <= kv_len" in _err(dsk)
    assert call(ld_tok=60) == 1 and "token stride" in _err(dsk)
    assert call(batch=2, ld_batch=640 * 63) == 1 and "batch" in _err(dsk)
    assert call(qa=(8192, 500)) == 3 and "multiples of 8" in _err(dsk)
    assert call(q_abs=None) == 2
    assert call(q_abs=24) == 3
    assert call(out=18) == 3
    assert call(kv_len=4096, bytes_=1024) == 5 and "workspace" in _err(dsk)
    assert call(batch=256, q_len=256, kv_len=256, ld_batch=640 * 256) == 1 and "65535" in _err(dsk)
    # k_rope is written while latent and k_pe are read: overlapping views are refused
    assert call(k_rope=kpe) == 1 and "overlaps" in _err(dsk)
    assert call(k_rope=lat + 512) == 1 and "overlaps" in _err(dsk)
    assert call(k_rope=lat + 1280 * 2, ld_tok=1280, ld_batch=1280 * 64) == 1  # next row's latent
    # columns 640..703 of 1280-wide rows: clear of both (stops at the workspace check)
    assert call(k_rope=lat + 1280 * 3, ld_tok=1280, ld_batch=1280 * 64, kv_len=4096,
                bytes_=1024) == 5
    assert call(k_rope=1 << 30, kv_len=4096, bytes_=1024) == 5  # a separate buffer


def test_linear_batched_validation(dsk):
    lib = dsk.lib
    # x, ld_x, x_batch_stride, w, out, ld_out, out_batch_stride, batch, M, K, N, stream
    rc = lib.dsk_linear_batched(16, 3072, 192, 16, 16, 2048, 128, 16, 65, 128, 512, None)
    assert rc == 1 and "64" in _err(dsk)
    rc = lib.dsk_linear_batched(16, 3072, 190, 16, 16, 2048, 128, 16, 1, 128, 512, None)
    assert rc == 3
    rc = lib.dsk_linear_batched(16, 3072, 0, 16, 16, 2048, 128, 16, 1, 128, 512, None)
    assert rc == 1 and "positive" in _err(dsk)
    rc = lib.dsk_linear_batched(16, 3072, 192, 16, 16, 2048, 128, 16, 1, 100, 512, None)
    assert rc == 1
    assert lib.dsk_linear_batched(None, 0, 0, None, None, 0, 0, 0, 1, 128, 512, None) == 0


def test_norm_rope_validation(dsk):
    lib = dsk.lib
    rc = lib.dsk_rms_norm(16, 511, 16, 16, 511, 4, 511, 1e-6, None)
    assert rc == 1 and "even" in _err(dsk)
    rc = lib.dsk_rope(16, 0, 0, 64, 16, 16, 0, 64, 16, 1, 1, 4, 60, None)
    assert rc == 1


def test_gate_validation(dsk):
    lib = dsk.lib
    rc = lib.dsk_moe_gate_logits(16, 2048, 16, None, 16, 65, 4, 65, 2048, 0, None)
    assert rc == 1 and "64" in _err(dsk)
    rc = lib.dsk_moe_gate_logits(16, 2048, 16, None, 16, 64, 4, 64, 2040, 0, None)
    assert rc == 1 and "16" in _err(dsk)
    rc = lib.dsk_moe_gate_logits(None, 2048, 16, None, 16, 64, 4, 64, 2048, 0, None)
    assert rc == 2
    rc = lib.dsk_moe_gate_logits(16, 2052, 16, None, 16, 64, 4, 64, 2048, 0, None)
    assert rc == 3
    rc = lib.dsk_moe_gate_logits(16, 2040, 16, None, 16, 64, 4, 64, 2048, 0, None)
    assert rc == 1 and "stride" in _err(dsk)
    rc = lib.dsk_moe_gate_logits(16, 2048, 16, None, 16, 40, 4, 40, 2048, 1, None)
    assert rc == 1 and "tiled" in _err(dsk)


def test_fused_validation_and_workspace_sizes(dsk):
    lib = dsk.lib
    assert lib.dsk_moe_fused_workspace_size(4096, 64, 6, 2, 2048, 1408) > \
        (4096 * 8) * (2048 + 1408) * 2
    assert lib.dsk_moe_dispatch_workspace_size(100, 64, 6) >= 2 * 100 * 6 * 4
    assert lib.dsk_moe_combine_workspace_size(600, 100) >= (2 * 101 + 2 * 600) * 4
    rc = lib.dsk_moe_fused_forward(None, None, None, None, None, 4, 64, 6, 2, 2048, 1400, 0,
                                   None, None, None, None, 0, None, None)
    assert rc == 1
    rc = lib.dsk_moe_fused_forward(16, 16, 16, 16, 16, 4, 64, 6, 2, 2048, 1408, 0, None, None,
                                   None, None, 0, None, None)
    assert rc == 5 and "workspace" in _err(dsk)
    rc = lib.dsk_moe_fused_forward(16, 16, 16, 16, 16, 4, 64, 6, 2, 2048, 1408, 7, None, None,
                                   None, None, 0, None, None)
    assert rc == 1 and "weight_layout" in _err(dsk)


def test_layer_forward_validation(dsk):
    lib = dsk.lib
    assert lib.dsk_moe_layer_workspace_size(16, 64, 6, 2, 2048, 1408) > \
        lib.dsk_moe_fused_workspace_size(16, 64, 6, 2, 2048, 1408)
    rc = lib.dsk_moe_layer_forward(16, 16, None, 16, 16, 16, 4, 40, 6, 2, 2048, 1408, 1,
                                   None, None, None, 16, 1 << 30, None, None)
    assert rc == 1 and "% 32" in _err(dsk)
    rc = lib.dsk_moe_layer_forward(16, None, None, 16, 16, 16, 4, 64, 6, 2, 2048, 1408, 1,
                                   None, None, None, 16, 1 << 30, None, None)
    assert rc == 2
    rc = lib.dsk_moe_layer_forward(16, 16, None, 16, 16, 16, 4, 64, 6, 2, 2048, 1408, 1,
                                   None, None, None, 16, 1024, None, None)
    assert rc == 5


def test_python_ops_reject_cpu_tensors(dsk):
    logits = torch.zeros(4, 64)
    with pytest.raises(RuntimeError, match="CUDA"):
        dsk.moe_routing(logits, 6)
    with pytest.raises(RuntimeError):
        dsk.moe_scan(torch.zeros(64, dtype=torch.int32))
    with pytest.raises(RuntimeError):
        dsk.rms_norm(torch.zeros(2, 8, dtype=torch.bfloat16), torch.ones(8))


def test_c_caller_links_and_calls(dsk, tmp_path):
    """A plain C99 caller (what a cgo / JNI / N-API stub compiles against):
    include/dsk.h compiles as C, links against libdsk.so, and the entry points
    answer without a GPU (version, a rejected argument and its message)."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "caller.c"
    src.write_text(r"""
#include <stdio.h>
#include <string.h>
#include "dsk.h"
int main(void) {
  if (dsk_abi_version() != 3) return 1;
  /* top_k = 7 is rejected before any device work */
  int rc = dsk_moe_routing(NULL, 64, NULL, NULL, NULL, 4, 64, 7, NULL, 0, NULL);
  if (rc != 1 || strstr(dsk_last_error(), "top_k") == NULL) return 2;
  printf("ok\n");
  return 0;
}
""")
    exe = tmp_path / "caller"
    libdir = os.path.dirname(dsk.LIB_PATH)
    subprocess.run([cc, "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    str(src), "-o", str(exe), os.path.join(libdir, "libdsk.so"),
                    "-Wl,-rpath," + libdir], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and out.stdout.strip() == "ok", (out.returncode, out.stderr)


def test_linear_row_statistics_validation(dsk):
    """The epilogue-RMSNorm pair rejects bad column ranges, missing statistics and
    empty reductions before any launch."""
    lib = dsk.lib
    # x, ld_x, w, out, ld_out, M, K, N, row_sumsq, ld_rowsq, c0, c1, stream
    def rowsq(c0=3072, c1=3584, ss=16, ld=8):
        return lib.dsk_linear_rowsq(16, 2048, 16, 16, 3648, 8, 2048, 3648, ss, ld, c0, c1, None)
    assert rowsq(ss=None) == 2 and "row_sumsq" in _err(dsk)
    assert rowsq(c0=3000) == 1 and "256-aligned" in _err(dsk)
    assert rowsq(c1=3840) == 1 and "256-aligned" in _err(dsk)
    assert rowsq(ld=4) == 1 and "ld_rowsq" in _err(dsk)
    # x, ld_x, w, out, ld_out, M, K, N, row_sumsq, ld_rowsq, n_parts, n_cols, eps, stream
    def rowscale(parts=2, cols=512, k=512):
        return lib.dsk_linear_rowscale(16, 576, 16, 16, 4096, 8, k, 4096, 16, 8, parts, cols,
                                       1e-6, None)
    assert rowscale(parts=0) == 1 and "parts" in _err(dsk)
    assert rowscale(parts=3) == 1 and "parts" in _err(dsk)
    assert rowscale(cols=0) == 1 and "cols" in _err(dsk)
    assert rowscale(k=64) == 1 and "K % 128" in _err(dsk)
