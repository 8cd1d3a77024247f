#!/usr/bin/env python3
"""Benchmark of the fused DeepSeek-V2-Lite MoE layer on one MI355X.

Headline (value): prefill MoE layer tokens/s at T=4096, bf16:
one step = dsk_moe_layer_forward: gate logits (bf16 products, fp32 accumulation) + the fused layer
(route -> permutation -> grouped GEMM1+SwiGLU -> grouped GEMM2 -> combine, the
2 shared experts included) over 4096 resident tokens.

Also reported on the same line:
  roofline      the dominant kernel (grouped GEMM1+SwiGLU), timed live with HIP
                events recorded by the library on the launch stream around that
                launch; achieved = algorithmic flops / mean duration vs the bf16
                dense MFMA peak. gemm2 / both GEMMs are given beside it.
  decode        T in {1, 4, 16, 64} with the Zipf-biased router (config 2): HBM
                GB/s of algorithmic bytes (touched expert weights + shared + gate +
                activations) per layer step, weights rotated over 4 copies so the
                256 MB MALL cannot serve them.
  mla           BASELINE configs 3 and 4: the MLA projection block (rms_norm on the
                strided latent, rope, kv_upproj, each timed by HIP-graph replay) and
                the decoder layer, composed from this library's kernels.
  cpu_baseline  the CPU oracle (numpy restatement of DeepSeekMoE.forward) timed
                on this host's cores: the same T=4096 workload (2 calls, fp32; the
                reported value) and config 0 (T=64) beside it.

Usage: python bench.py [--gpus 1] [--steps K (200)] [--warmup W (20)]
                       [--profile | --decode-only T | --mla-only | --mla-decode-only | --ramp]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deepseek-v2-lite-cuda_amd"))

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
METRIC = "MoE layer tokens/s bf16 at T=4096 (MFMA %); T=16 decode HBM GB/s (% of 8TB/s)"


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hipEventDisableSystemFence (hip_runtime_api.h)


class HipEvents:
    """Raw hipEvent_t handles from the HIP runtime torch already loaded. They are
    timing-only events (hipEventDisableSystemFence): recording one does not write
    back and invalidate the caches as a default event does, which cost ~2 us of GPU
    time per event and ~6 us per instrumented layer step (722.7 against 729.1 us,
    no events at all 721.8 us). Elapsed times are read after a device
    synchronisation."""

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so.7")
        self.rt.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.rt.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]

    def create(self, n):
        arr = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            if self.rt.hipEventCreateWithFlags(ctypes.byref(h),
                                               HIP_EVENT_DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            arr[i] = h
        return arr

    def ms(self, a, b):
        f = ctypes.c_float()
        if self.rt.hipEventElapsedTime(ctypes.byref(f), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return f.value

    def destroy(self, arr):
        for h in arr:
            self.rt.hipEventDestroy(h)


def bench_prefill(dsk, syn, torch, F, W, packed, T, steps, warmup, ev):
    """The headline steps. Inside the timed region the library records three HIP
    events per step on the launch stream: before GEMM1, after GEMM1 and after
    GEMM2 (timing-only events; only the ones the roofline needs are recorded, so
    the instrumented steps run as fast as uninstrumented ones). They give GEMM1's and GEMM2's
    launch times and the step period (consecutive GEMM1 starts). The gate+route
    and combine stage times come from 10 further steps with all five stage events,
    after the timed region."""
    w1, w2, nsh = packed
    dev = w1.device
    wg = dsk.tile_weights(W.wg.to(torch.bfloat16)[None])[0].to(dev)   # fragment-tiled gate
    x = syn.tokens(T).to(torch.bfloat16).to(dev)
    H, I = 2048, 1408
    ws = torch.empty(dsk.lib.dsk_moe_layer_workspace_size(T, 64, 6, nsh, H, I),
                     dtype=torch.uint8, device=dev)
    timed_ev = [ev.create(3) for _ in range(steps)]
    events = []
    for e in timed_ev:   # stage slots 1..3; slots 0 and 4 (before the gate, after the combine) empty
        arr = (ctypes.c_void_p * 5)()
        arr[1], arr[2], arr[3] = e[0], e[1], e[2]
        events.append(arr)

    def step(e=None):
        return dsk.moe_layer_forward(x, wg, w1, w2, 6, nsh, workspace=ws, stage_events=e)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(events[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    g1 = [ev.ms(e[0], e[1]) for e in timed_ev]
    g2 = [ev.ms(e[1], e[2]) for e in timed_ev]
    period = sorted(ev.ms(timed_ev[i][0], timed_ev[i + 1][0]) for i in range(steps - 1))
    for e in timed_ev:
        ev.destroy(e)
    full = [ev.create(5) for _ in range(10)]
    for e in full:
        step(e)
    torch.cuda.synchronize()
    stage = [[ev.ms(e[j], e[j + 1]) for j in range(4)] for e in full]
    for e in full:
        ev.destroy(e)
    mean = lambda v: sum(v) / len(v)  # noqa: E731
    med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
    return {
        "ms_per_step": elapsed * 1e3 / steps,
        "step_ms_median": period[len(period) // 2] if period else None,
        "step_ms_p95": period[min(len(period) - 1, int(0.95 * len(period)))] if period else None,
        "gemm1_ms": mean(g1),
        "gemm2_ms": mean(g2),
        "gate_route_ms_after_timed_steps": med([s_[0] for s_ in stage]),
        "combine_ms_after_timed_steps": med([s_[3] for s_ in stage]),
        "rows": T * 6 + nsh * T,
    }


def bench_decode(dsk, syn, torch, F, W, packed, T, steps, ev, copies):
    w1, w2, nsh = packed
    dev = w1.device
    wg = dsk.tile_weights(W.wg.to(torch.bfloat16)[None])[0].to(dev)   # fragment-tiled gate
    bias = syn.zipf_router_bias().to(dev)
    x = syn.tokens(T).to(torch.bfloat16).to(dev)
    H, I = 2048, 1408
    ws = torch.empty(dsk.lib.dsk_moe_layer_workspace_size(T, 64, 6, nsh, H, I),
                     dtype=torch.uint8, device=dev)

    def step(c):
        return dsk.moe_layer_forward(x, wg, copies[c][0], copies[c][1], 6, nsh, gate_bias=bias,
                                     workspace=ws)

    _, (idx, _, off) = dsk.moe_layer_forward(x, wg, w1, w2, 6, nsh, gate_bias=bias,
                                             return_routing=True)
    counts = (off[1:] - off[:-1]).cpu()
    e_active = int((counts > 0).sum())
    for i in range(5):
        step(i % len(copies))
    torch.cuda.synchronize()

    def timed(run):
        evs = ev.create(2 * steps)
        st = torch.cuda.current_stream().cuda_stream
        for i in range(steps):
            ev.rt.hipEventRecord(evs[2 * i], st)
            run(i % len(copies))
            ev.rt.hipEventRecord(evs[2 * i + 1], st)
        torch.cuda.synchronize()
        times = sorted(ev.ms(evs[2 * i], evs[2 * i + 1]) for i in range(steps))
        ev.destroy(evs)
        return times[len(times) // 2]

    # eager: one Python call (5 kernel launches) per step. Graph: the same step
    # captured once per weight copy and replayed one step per launch, and ten
    # steps (cycling the copies) captured in one graph. Launching a graph costs a
    # fixed ~6-7 us on MI355X, whatever it holds; its kernel nodes add nothing
    # (ten captured steps run faster per step than eager ones), so the one-step
    # replay is the slowest form and the ten-step graph the fastest.
    med_eager = timed(step)
    graphs = []
    for c in range(len(copies)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(c)
        graphs.append(g)
    g10 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g10):
        for j in range(10):
            step(j % len(copies))
    for i in range(3):
        graphs[i % len(graphs)].replay()
        g10.replay()
    torch.cuda.synchronize()
    med_graph = timed(lambda c: graphs[c].replay())
    med_graph10 = timed(lambda c: g10.replay()) / 10
    del graphs, g10
    med = med_eager
    bytes_ = e_active * (3 * I * H * 2) + nsh * (3 * I * H * 2) + 64 * H * 2 + 2 * T * H * 2
    gbs = bytes_ / (med * 1e-3) / 1e9
    return {"tokens": T, "E_active": e_active, "us_per_step": med * 1e3,
            "us_per_step_graph_replay": med_graph * 1e3,
            "us_per_step_graph_of_10_steps": med_graph10 * 1e3,
            "timing": "median of 50 eager steps, HIP events on the launch stream",
            "algorithmic_bytes": bytes_, "GB/s": gbs, "frac_of_8TB/s": gbs / PEAK_HBM_GBS}


def ramp_probe(dsk, syn, torch, W, packed, ev, n=60):
    """Per-step times of the T=4096 layer right after the set-up (no warm-up), then,
    after one idle second each: 40 launches of a 512 MB device copy (HBM only),
    40 of a dense 8192^3 bf16 product (matrix cores only) and 30 more layer
    steps. A core-clock ramp slows the product and the layer, not the copy."""
    w1, w2, nsh = packed
    dev = w1.device
    wg = dsk.tile_weights(W.wg.to(torch.bfloat16)[None])[0].to(dev)
    x = syn.tokens(4096).to(torch.bfloat16).to(dev)
    ws = torch.empty(dsk.lib.dsk_moe_layer_workspace_size(4096, 64, 6, nsh, 2048, 1408),
                     dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream

    def layer_steps(k):
        evs = [ev.create(5) for _ in range(k)]
        for e in evs:
            dsk.moe_layer_forward(x, wg, w1, w2, 6, nsh, workspace=ws, stage_events=e)
        torch.cuda.synchronize()
        out = [[ev.ms(e[j], e[j + 1]) * 1e3 for j in range(4)] for e in evs]
        for e in evs:
            ev.destroy(e)
        return out

    def launches(fn, k):
        evs = ev.create(2 * k)
        for i in range(k):
            ev.rt.hipEventRecord(evs[2 * i], st)
            fn()
            ev.rt.hipEventRecord(evs[2 * i + 1], st)
        torch.cuda.synchronize()
        out = [ev.ms(evs[2 * i], evs[2 * i + 1]) * 1e3 for i in range(k)]
        ev.destroy(evs)
        return out

    res = {"layer_steps_after_setup_us": layer_steps(n)}
    src = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    a = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    b = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    c = torch.empty_like(a)
    torch.mm(a, b, out=c)
    torch.cuda.synchronize()
    time.sleep(1.0)
    res["copy_512MB_after_idle_us"] = launches(lambda: dst.copy_(src), 40)
    time.sleep(1.0)
    res["mm_8192_bf16_after_idle_us"] = launches(lambda: torch.mm(a, b, out=c), 40)
    time.sleep(1.0)
    res["layer_steps_after_idle_us"] = layer_steps(30)
    return res


def graph_timer(torch, ev, reps=20, warmup=5):
    """Returns timed(fn, per_graph=10): the median time of fn on the GPU, with
    per_graph back-to-back calls captured in a HIP graph (so host-side Python cost
    between launches does not leave the GPU idle), replayed `reps` times between
    HIP events on the stream."""
    def timed(fn, per_graph=10):
        st = torch.cuda.current_stream().cuda_stream
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(per_graph):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        evs = ev.create(2 * reps)
        for i in range(reps):
            ev.rt.hipEventRecord(evs[2 * i], st)
            graph.replay()
            ev.rt.hipEventRecord(evs[2 * i + 1], st)
        torch.cuda.synchronize()
        t = sorted(ev.ms(evs[2 * i], evs[2 * i + 1]) / per_graph for i in range(reps))
        ev.destroy(evs)
        del graph
        return t[len(t) // 2]
    return timed


def bench_mla(dsk, syn, torch, ev, reps=20, warmup=5):
    """BASELINE configs 3 and 4: the MLA projection block at 8 x 2048 (rms_norm and
    rope against HBM, kv_upproj against MFMA, each timed with HIP events on the
    launch stream) and the full decoder layer at 4 x 2048 (tokens/s)."""
    from ds_kernels import mla as dm
    dev = torch.device("cuda:0")
    W = dm.MLAWeights.from_tensors(syn.mla_weights(), dev)
    b, s, H = 8, 2048, 2048
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(b, s, H, generator=g).to(torch.bfloat16).to(dev)
    cos, sin = dm.yarn_cos_sin(s, device=dev)
    cb = cos.to(torch.bfloat16)[None, None].expand(b, 1, s, 64)
    sb = sin.to(torch.bfloat16)[None, None].expand(b, 1, s, 64)
    q = dsk.linear(x, W.q).view(b, s, 16, 192).transpose(1, 2)
    kva = dsk.linear(x, W.kva)
    latent = dsk.rms_norm(kva[..., :512], W.kva_norm)
    k_pe = kva[..., 512:].view(b, s, 1, 64).transpose(1, 2)
    timed = graph_timer(torch, ev, reps, warmup)
    rows = b * s
    t_norm = timed(lambda: dsk.rms_norm(kva[..., :512], W.kva_norm))
    t_rope = timed(lambda: dsk.rope(q[..., 128:], k_pe, cb, sb))
    t_kvb = timed(lambda: dsk.kv_upproj(latent, W.kvb))      # tiled weight (the block's)
    kvb_rm = dsk.untile_weights(W.kvb[None])[0].contiguous()
    t_kvb_rm = timed(lambda: dsk.kv_upproj(latent, kvb_rm))  # reference layout
    # the block as the reference computes it (q, k, v; the latent norm riding the
    # q/kv_a and kv_b epilogues), and beside it with the norm as a separate pass
    t_block = timed(lambda: dm.mla_projections(x, W, cos, sin, with_latent=False))
    import dataclasses
    W_sep = dataclasses.replace(W, kvb_w=None)
    t_block_sep = timed(lambda: dm.mla_projections(x, W_sep, cos, sin))
    t_qkva = timed(lambda: dsk.linear(x, W.q_kva))
    t_qkva_sq = timed(lambda: dsk.linear_rowsq(x, W.q_kva, 3072, 3584))
    _, ss = dsk.linear_rowsq(x, W.q_kva, 3072, 3584)
    t_kvb_rs = timed(lambda: dsk.linear_rowscale(kva[..., :512], W.kvb_w, ss, 512))
    norm_bytes = 2 * rows * 512 * 2 + 512 * 4
    rope_bytes = 2 * (rows * 16 * 64 * 2) + 2 * (rows * 64 * 2) + 2 * (s * 64 * 2)
    # the practical ceiling at these sizes: a device-to-device copy of the same
    # number of bytes (half read, half written), by HIP-graph replay like the kernels
    def copy_us(nbytes):
        src = torch.empty(nbytes // 2, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        return timed(lambda: dst.copy_(src)) * 1e3
    cp_norm, cp_rope = copy_us(norm_bytes), copy_us(rope_bytes)
    kvb_flops = 2.0 * rows * 512 * 4096
    kvb_bytes = rows * 512 * 2 + 4096 * 512 * 2 + rows * 4096 * 2
    gbs = lambda nbytes, ms: nbytes / (ms * 1e-3) / 1e9  # noqa: E731
    out = {
        "config3_projection_block": {
            "shape": "b=8, s=2048: q 2048->3072, kv_a 2048->576, rms_norm(512, strided), "
                     "kv_b 512->4096, rope(q 16 heads + k, 64 dims)",
            "block_ms": t_block, "tokens_per_s": rows / (t_block * 1e-3),
            "block_ms_norm_as_separate_pass": t_block_sep,
            "latent_norm_in_epilogues": {
                "q_kva_us": t_qkva * 1e3, "q_kva_with_row_sumsq_us": t_qkva_sq * 1e3,
                "kv_b_us": t_kvb * 1e3, "kv_b_with_row_scale_us": t_kvb_rs * 1e3,
                "rms_norm_pass_us": t_norm * 1e3},
            "rms_norm": {"us": t_norm * 1e3, "algorithmic_bytes": norm_bytes,
                         "GB/s": gbs(norm_bytes, t_norm),
                         "frac_of_8TB/s": gbs(norm_bytes, t_norm) / PEAK_HBM_GBS,
                         "same_bytes_device_copy_us": cp_norm},
            "rope": {"us": t_rope * 1e3, "algorithmic_bytes": rope_bytes,
                     "GB/s": gbs(rope_bytes, t_rope),
                     "frac_of_8TB/s": gbs(rope_bytes, t_rope) / PEAK_HBM_GBS,
                     "same_bytes_device_copy_us": cp_rope},
            "kv_upproj": {"us": t_kvb * 1e3, "flops": kvb_flops,
                          "TFLOP/s": kvb_flops / (t_kvb * 1e-3) / 1e12,
                          "frac_of_bf16_peak": kvb_flops / (t_kvb * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                          "GB/s": gbs(kvb_bytes, t_kvb), "weight_layout": "fragment-tiled",
                          "us_row_major_weight": t_kvb_rm * 1e3},
        }}
    del q, kva, latent, k_pe, ss
    # config 4: the decoder layer at 4 x 2048
    P = dm.DecoderLayerWeights.from_tensors(syn.mla_weights(), syn.moe_weights(), dev)
    b4 = 4
    x4 = torch.randn(b4, s, H, generator=g).to(torch.bfloat16).to(dev)
    t_layer = timed(lambda: dm.decoder_layer_forward(x4, P, cos, sin), per_graph=2)
    out["config4_decoder_layer"] = {
        "shape": "b=4, s=2048, causal; MLA (16 heads) + MoE (64 routed top-6 + 2 shared)",
        "layer_ms": t_layer, "tokens_per_s": b4 * s / (t_layer * 1e-3)}
    del P, x4
    out["latent_cache_decode"] = bench_latent_decode(dsk, torch, dm, W, timed, dev, g)
    return out


def bench_latent_decode(dsk, torch, dm, W, timed, dev, g):
    """Decode over the latent KV cache: the attention op alone (reads every
    cached token's latent and rotated RoPE key, 1152 bytes, once; HBM-bound) at
    a few (batch, cache length) points, and one whole decode step (projections,
    cache append, absorbed attention, W_UV, o_proj) for one new token after
    4095 cached ones, beside the full-sequence recompute at 4096 that a
    cache-less forward pays. The op is timed over enough copies of the cache
    (at least 512 MB, cycled in order) that no call finds its rows in the
    256 MB Infinity Cache, as a layer of a real model would not; each call
    rotates its n new keys itself (rope_len = L - n), as in a decode step."""
    from ds_kernels import ops
    A = dsk.AbsorbedMLAWeights.from_mla(W)
    cos, sin = dm.yarn_cos_sin(8192, device=dev)
    cos, sin = cos.to(torch.bfloat16), sin.to(torch.bfloat16)
    gbs = lambda nbytes, ms: nbytes / (ms * 1e-3) / 1e9  # noqa: E731
    res = {"attention_op": []}
    for b, L, n in ((1, 4096, 1), (4, 4096, 1), (16, 4096, 1), (1, 4096, 8)):
        raw = torch.randn(b, L, 576, generator=g).to(torch.bfloat16).to(dev)
        rows = torch.zeros(b, L, 640, dtype=torch.bfloat16, device=dev)   # LatentKVCache rows
        rows[..., :576] = raw
        c = cos[:L][None, None].expand(b, 1, L, 64)
        sn = sin[:L][None, None].expand(b, 1, L, 64)
        rows[..., 576:] = ops.rope_single(raw[:, None, :, 512:], c, sn)[:, 0]
        copies = max(2, min(64, -(-(512 << 20) // (rows.numel() * 2))))
        bufs = [rows] + [rows.clone() for _ in range(copies - 1)]
        q_abs = (torch.randn(b * n, 16, 512, generator=g) * 0.05).to(torch.bfloat16).to(dev)
        q_pe = torch.randn(b * n, 16, 64, generator=g).to(torch.bfloat16).to(dev)
        o = torch.empty(b * n, 16, 512, dtype=torch.bfloat16, device=dev)
        nxt = [0]

        def call():
            r = bufs[nxt[0] % copies]
            nxt[0] += 1
            dsk.mla_decode_attention(q_abs, q_pe, r[..., :512], r[..., 512:576], cos, sin,
                                     W.softmax_scale, out=o, k_rope=r[..., 576:],
                                     rope_len=L - n)
        t = timed(call, per_graph=copies)
        nbytes = b * L * 576 * 2 + 2 * b * n * 16 * (512 + 64 + 512)
        res["attention_op"].append({"batch": b, "cache_len": L, "new_tokens": n, "us": t * 1e3,
                                    "algorithmic_bytes": nbytes, "GB/s": gbs(nbytes, t),
                                    "frac_of_8TB/s": gbs(nbytes, t) / PEAK_HBM_GBS,
                                    "cache_copies": copies})
        del raw, rows, bufs, q_abs, q_pe, o
    L = 4096
    x = torch.randn(1, L, 2048, generator=g).to(torch.bfloat16).to(dev)
    cache = dsk.LatentKVCache.for_inference(1, max_seq=L, device=dev)
    dsk.mla_decode_forward(x[:, :L - 1], W, cache, cos, sin, A)   # prefix into the cache
    x1 = x[:, L - 1:].contiguous()

    def step():
        cache._len = L - 1          # re-append position L-1 each call
        dsk.mla_decode_forward(x1, W, cache, cos, sin, A)

    t_step = timed(step)
    # four sequences at once: one new token each (the few-row projections at 4 rows)
    x4 = torch.randn(4, L, 2048, generator=g).to(torch.bfloat16).to(dev)
    cache4 = dsk.LatentKVCache.for_inference(4, max_seq=L, device=dev)
    dsk.mla_decode_forward(x4[:, :L - 1], W, cache4, cos, sin, A)
    x41 = x4[:, L - 1:].contiguous()

    def step4():
        cache4._len = L - 1
        dsk.mla_decode_forward(x41, W, cache4, cos, sin, A)

    t_step4 = timed(step4)
    del x4, cache4, x41
    cf, sf = dm.yarn_cos_sin(L, device=dev)
    t_full = timed(lambda: dm.mla_forward(x, W, cf, sf), per_graph=1)
    res["decode_step"] = {"batch": 1, "cache_len": L, "us": t_step * 1e3,
                          "full_sequence_recompute_us": t_full * 1e3,
                          "note": "one new token: q / kv_a projections, cache append, absorbed "
                                  "attention, W_UV, o_proj; versus mla_forward over all 4096 "
                                  "positions (what a forward without a cache recomputes)"}
    res["decode_step_b4"] = {"batch": 4, "cache_len": L, "us": t_step4 * 1e3,
                             "note": "one new token in each of 4 sequences, same step"}
    return res


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(W, syn, budget_s):
    """The CPU oracle (numpy fp32 restatement of DeepSeekMoE.forward, reference
    src/reference/moe.py:77-109) on this host: the same workload as the GPU line
    (T=4096, 2 timed calls after one warm-up) and config 0 (T=64, calls until
    budget_s). `value` is the T=4096 rate."""
    import numpy as np
    from oracle import moe as om
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info()
                       if p.get("user_api") == "blas"] or [1])
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    wts = (W.wg.numpy(), W.gates.numpy(), W.ups.numpy(), W.downs.numpy())
    shared = tuple(t.numpy() for t in W.shared)

    def rate(T, min_calls, max_calls, budget):
        x = syn.tokens(T).numpy()
        om.moe_layer(x, *wts, 6, shared=shared)          # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            om.moe_layer(x, *wts, 6, shared=shared)
            n += 1
            el = time.perf_counter() - t0
            if (el >= budget and n >= min_calls) or n >= max_calls:
                return T * n / el, n, el

    v4096, n4096, e4096 = rate(4096, 2, 2, 0.0)
    v64, n64, e64 = rate(64, 2, 200, budget_s)
    model = _cpu_model()
    return {"value": v4096, "unit": "tokens/s", "cores": int(threads), "kind": "port",
            "sample": f"oracle DeepSeekMoE.forward restatement (numpy fp32) on {model}: "
                      f"T=4096 (the GPU line's workload) {n4096} calls in {e4096:.1f} s; "
                      f"config 0 T=64 {n64} calls in {e64:.1f} s; BLAS threads={threads}, "
                      f"os.cpu_count()={os.cpu_count()}",
            "tokens_per_s_T4096": v4096, "tokens_per_s_T64": v64, "cpu_model": model,
            "blas_threads": int(threads), "os_cpu_count": os.cpu_count()}


COPY_BYTES = 1 << 30  # calibration copy: 1 GiB read + 1 GiB written per launch


def calibrate_copy(steps):
    """Plain device copy of COPY_BYTES, the reference kernel for the HBM counters:
    FETCH_SIZE / WRITE_SIZE of the GEMM are scaled by what the counters read here
    against the known 1 GiB."""
    import torch
    src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda:0").normal_()
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "launches": steps}), flush=True)


def dense_gemm2(dsk, torch, reps):
    """GEMM2's shape as one dense product (32768 x 2048 x 1408, bf16): torch's
    library GEMM (hipBLASLt) against this build's weight-streaming kernel on the
    fragment-tiled weight, same inputs; for timing and counter passes."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    M, N, K = 32768, 2048, 1408
    a = torch.randn(M, K, device=dev, dtype=torch.bfloat16, generator=g)
    w = torch.randn(N, K, device=dev, dtype=torch.bfloat16, generator=g)
    wt = dsk.tile_weights(w[None])[0].contiguous()
    for _ in range(10):
        y_lib = torch.nn.functional.linear(a, w)
        y_dsk = dsk.linear(a, wt)
    torch.cuda.synchronize()
    res = {"shape": [M, N, K], "max_abs_diff": (y_lib.float() - y_dsk.float()).abs().max().item()}
    for name, f in (("hipblaslt_us", lambda: torch.nn.functional.linear(a, w)),
                    ("dsk_linear_us", lambda: dsk.linear(a, wt))):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            f()
        e.record()
        torch.cuda.synchronize()
        res[name] = s.elapsed_time(e) / reps * 1e3
    return res


def _pmc_per_dispatch(csv_path, kernel_substrs, counter):
    import csv
    vals = {}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            if (all(k in r["Kernel_Name"] for k in kernel_substrs)
                    and r["Counter_Name"].startswith(counter)):
                vals[r["Dispatch_Id"]] = vals.get(r["Dispatch_Id"], 0.0) + float(
                    r["Counter_Value"])
    return sorted(vals.values())


def summarize_traffic(gemm_fetch, gemm_write, copy_fetch, copy_write, out_path):
    """HBM bytes per launch of the SwiGLU GEMM from rocprofv3 --pmc CSVs
    (FETCH_SIZE and WRITE_SIZE passes over `bench.py --profile` and over
    `bench.py --calibrate-copy`), each scaled by the copy's counter/byte ratio."""
    kib = 1024.0
    med = lambda v: v[len(v) // 2]  # noqa: E731
    cf = _pmc_per_dispatch(copy_fetch, (), "FETCH_SIZE")
    cw = _pmc_per_dispatch(copy_write, (), "WRITE_SIZE")
    # the copy is the only large kernel in its run: take its biggest dispatch
    f_scale = COPY_BYTES / (max(cf) * kib)
    w_scale = COPY_BYTES / (max(cw) * kib)
    swiglu_gather = ("grouped_gemm_kernel", "true, true>")  # SWIGLU, GATHER
    gf = med(_pmc_per_dispatch(gemm_fetch, swiglu_gather, "FETCH_SIZE"))
    gw = med(_pmc_per_dispatch(gemm_write, swiglu_gather, "WRITE_SIZE"))
    res = {"kernel": "grouped_gemm_kernel SwiGLU+gather (gemm1), T=4096",
           "fetch_kib_raw": gf, "write_kib_raw": gw,
           "fetch_scale": f_scale, "write_scale": w_scale,
           "hbm_read_bytes": gf * kib * f_scale, "hbm_write_bytes": gw * kib * w_scale,
           "hbm_bytes_per_launch": gf * kib * f_scale + gw * kib * w_scale}
    with open(out_path, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res))


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-traffic":
        summarize_traffic(*sys.argv[2:7])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 20 warm-up + 200 timed steps, as the reference's benchmark
    # (tests/benchmark_moe_performance.py:50-51); after a cold start the layer
    # step takes ~15 steps to settle (clocks and caches)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--decode-steps", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile", action="store_true",
                    help="prefill steps only (no decode sweep, no CPU baseline)")
    ap.add_argument("--decode-only", type=int, default=0, metavar="T",
                    help="only the decode-shaped layer at T tokens (for profiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only the 1 GiB device copy used to scale the HBM counters")
    ap.add_argument("--mla-only", action="store_true",
                    help="only the MLA projection block and decoder layer (for profiling)")
    ap.add_argument("--mla-decode-only", action="store_true",
                    help="only the latent-cache decode attention and decode step (for profiling)")
    ap.add_argument("--dense-gemm2", type=int, default=0, metavar="REPS",
                    help="GEMM2's shape as a dense product: the library GEMM against "
                         "dsk_linear_ex, REPS timed calls each")
    ap.add_argument("--ramp", action="store_true",
                    help="per-step layer times from a cold start, and a copy and a dense product "
                         "after an idle second (the clock ramp)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy(3)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only, see the sharding section of the docs)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import torch.nn.functional as F
    import ds_kernels as dsk
    from ds_kernels import synthetic as syn

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.mla_only:
        print(json.dumps(bench_mla(dsk, syn, torch, HipEvents())), flush=True)
        return
    if args.dense_gemm2:
        print(json.dumps(dense_gemm2(dsk, torch, args.dense_gemm2)), flush=True)
        return
    if args.mla_decode_only:
        from ds_kernels import mla as dm
        W = dm.MLAWeights.from_tensors(syn.mla_weights(), dev)
        timed = graph_timer(torch, HipEvents())
        print(json.dumps(bench_latent_decode(dsk, torch, dm, W, timed, dev,
                                             torch.Generator().manual_seed(1234))), flush=True)
        return
    print("bench: generating synthetic weights", file=sys.stderr, flush=True)
    W = syn.moe_weights()
    w1, w2, nsh = dsk.pack_tensors(W.gates, W.ups, W.downs, device=dev, shared=W.shared)
    # the fused layer's native layout: fragment-tiled expert weights
    packed = (dsk.tile_weights(w1), dsk.tile_weights(w2), nsh)
    del w1, w2
    ev = HipEvents()

    if args.ramp:
        print(json.dumps(ramp_probe(dsk, syn, torch, W, packed, ev)), flush=True)
        return

    if args.decode_only:
        w1, w2, nsh = packed
        copies = [(w1, w2)] + [(w1.clone(), w2.clone()) for _ in range(3)]
        print(json.dumps(bench_decode(dsk, syn, torch, F, W, packed, args.decode_only,
                                      args.decode_steps, ev, copies)), flush=True)
        return

    print("bench: prefill", file=sys.stderr, flush=True)
    pre = bench_prefill(dsk, syn, torch, F, W, packed, args.tokens, args.steps, args.warmup, ev)
    T = args.tokens
    rows = pre["rows"]
    H, I = 2048, 1408
    flops_g1 = 2.0 * rows * (2 * I) * H
    flops_g2 = 2.0 * rows * I * H
    ach_g1 = flops_g1 / (pre["gemm1_ms"] * 1e-3) / 1e12
    ach_g2 = flops_g2 / (pre["gemm2_ms"] * 1e-3) / 1e12
    ach_both = (flops_g1 + flops_g2) / ((pre["gemm1_ms"] + pre["gemm2_ms"]) * 1e-3) / 1e12
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "gemm1_swiglu_T4096_traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": T / (pre["ms_per_step"] * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) weights, N(0,1) activations, cast to bf16",
        "config": {"workload": "moe_layer_prefill", "tokens": T, "hidden": H,
                   "routed_experts": 64, "top_k": 6, "shared_experts": 2,
                   "intermediate": I, "parallelism": "single-gpu"},
        "roofline": {"kernel": "grouped_gemm1_swiglu", "bound": "mfma", "achieved": ach_g1,
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": ach_g1 / PEAK_BF16_TFLOPS, "traffic": traffic,
                     "flops_per_launch": flops_g1, "mean_launch_ms": pre["gemm1_ms"]},
        "stages_ms": {k: pre[k] for k in ("gemm1_ms", "gemm2_ms", "step_ms_median", "step_ms_p95",
                                          "gate_route_ms_after_timed_steps",
                                          "combine_ms_after_timed_steps")},
        "gemm2": {"achieved_tflops": ach_g2, "frac": ach_g2 / PEAK_BF16_TFLOPS},
        "gemms_combined": {"achieved_tflops": ach_both, "frac": ach_both / PEAK_BF16_TFLOPS},
    }
    if not args.profile:
        print("bench: decode sweep", file=sys.stderr, flush=True)
        w1, w2, nsh = packed
        copies = [(w1, w2)] + [(w1.clone(), w2.clone()) for _ in range(3)]
        out["decode"] = [bench_decode(dsk, syn, torch, F, W, packed, t, args.decode_steps, ev,
                                      copies) for t in (1, 4, 16, 64)]
        del copies
        print("bench: mla block and decoder layer", file=sys.stderr, flush=True)
        out["mla"] = bench_mla(dsk, syn, torch, ev)
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(W, syn, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
