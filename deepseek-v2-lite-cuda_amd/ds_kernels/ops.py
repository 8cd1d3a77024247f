"""Torch-facing ops of ds_kernels: same names, argument order, defaults and
return structure as the reference pybind module (src/kernels/bindings.cu:77-192).

Every op checks its inputs the way the reference wrapper does (device, dtype,
rank, contiguity: TORCH_CHECK -> RuntimeError), allocates its outputs and
workspaces with the torch allocator on the input's device, and launches on
torch's current stream through libdsk.so. There is no CPU path: CPU tensors are
rejected, and a missing library fails at import.
"""
from __future__ import annotations

from typing import List

import torch

from ._lib import check, lib, stream_handle

MAX_EXPERTS = 64
MAX_TOP_K = 6


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _cuda_contig(t: torch.Tensor, name: str, op: str) -> None:
    _req(isinstance(t, torch.Tensor), f"{op}: {name} must be a tensor.")
    _req(t.is_cuda, f"{op}: {name} must reside on a CUDA device.")
    _req(t.is_contiguous(), f"{op}: {name} must be contiguous in memory.")


def _dtype(t: torch.Tensor, dt: torch.dtype, name: str, op: str) -> None:
    _req(t.dtype == dt, f"{op}: {name} must be of type {str(dt).replace('torch.', '')}.")


def _ws(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# -------------------------------------------------------------- gate logits --
def moe_gate(x: torch.Tensor, weight: torch.Tensor,
             bias: "torch.Tensor | None" = None) -> torch.Tensor:
    """Router logits fp32 [T, E] = x @ weight^T (+ bias), bf16 in, fp32 accumulation.

    Replaces F.linear(x.float(), weight.float()) (moe_fused.py:131, moe.py:35-37);
    bias (fp32 [E]) is an optional per-expert routing bias added to the logits."""
    op = "moe_gate"
    _req(x.is_cuda and weight.is_cuda, f"{op}: x and weight must be CUDA tensors.")
    _dtype(x, torch.bfloat16, "x", op)
    _dtype(weight, torch.bfloat16, "weight", op)
    _req(x.dim() == 2 and x.stride(1) == 1, f"{op}: x must be [tokens, hidden] with unit column stride.")
    _cuda_contig(weight, "weight", op)
    T, H = x.shape
    tiled = weight.dim() == 4   # [E/32, H/16, 64, 8] from tile_weights(w[None])[0]
    if tiled:
        _req(tuple(weight.shape[2:]) == (64, 8) and weight.shape[1] * 16 == H,
             f"{op}: tiled weight must be [experts/32, {H // 16}, 64, 8].")
        E = weight.shape[0] * 32
    else:
        E = weight.shape[0]
        _req(weight.dim() == 2 and weight.shape[1] == H, f"{op}: weight must be [experts, {H}].")
    _req(E <= MAX_EXPERTS, "num_experts must not exceed 64.")
    if bias is not None:
        _cuda_contig(bias, "bias", op)
        _dtype(bias, torch.float32, "bias", op)
        _req(tuple(bias.shape) == (E,), f"{op}: bias must be [{E}].")
    dev = x.device
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(lib.dsk_moe_gate_logits(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                      bias.data_ptr() if bias is not None else None,
                                      logits.data_ptr(), E, T, E, H, 1 if tiled else 0,
                                      stream_handle(dev)), op)
    return logits


# ----------------------------------------------------------------- routing --
def moe_routing(logits: torch.Tensor, top_k: int = 6) -> List[torch.Tensor]:
    """Fused softmax + top-k routing (routing.cu:266-301).

    logits fp32 [T, E] -> [topk_indices int32 [T,K], topk_weights fp32 [T,K],
    expert_counts int32 [E]]. Ties go to the lower expert index; the k entries
    are in descending weight order."""
    op = "moe_routing"
    _cuda_contig(logits, "logits", op)
    _dtype(logits, torch.float32, "logits", op)
    _req(logits.dim() == 2, f"{op}: logits must be a 2-D tensor [tokens, experts].")
    T, E = logits.shape
    _req(E <= MAX_EXPERTS, "num_experts must not exceed 64.")
    _req(top_k <= MAX_TOP_K, "top_k must not exceed 6.")
    _req(top_k >= 1 and top_k <= E, f"{op}: top_k must be in [1, num_experts].")
    dev = logits.device
    idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    counts = torch.empty((E,), dtype=torch.int32, device=dev)
    nws = lib.dsk_moe_routing_workspace_size(T, E)
    ws = _ws(nws, dev)
    with torch.cuda.device(dev):
        check(lib.dsk_moe_routing(logits.data_ptr(), E, idx.data_ptr(), w.data_ptr(),
                                  counts.data_ptr(), T, E, top_k, ws.data_ptr(), ws.numel(),
                                  stream_handle(dev)), op)
    return [idx, w, counts]


def moe_scan(expert_counts: torch.Tensor) -> torch.Tensor:
    """Exclusive prefix sum with sentinel (scan.cu:86-130), entirely on the device."""
    op = "moe_scan"
    _cuda_contig(expert_counts, "expert_counts", op)
    _dtype(expert_counts, torch.int32, "expert_counts", op)
    _req(expert_counts.dim() == 1, f"{op}: expert_counts must be a 1-D tensor [num_experts].")
    E = expert_counts.shape[0]
    _req(1 <= E <= MAX_EXPERTS, f"{op}: num_experts must be in [1, 64].")
    dev = expert_counts.device
    offsets = torch.empty((E + 1,), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        check(lib.dsk_moe_scan(expert_counts.data_ptr(), offsets.data_ptr(), E,
                               stream_handle(dev)), op)
    return offsets


def moe_dispatch(input: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                 expert_offsets: torch.Tensor) -> List[torch.Tensor]:
    """Stable dispatch (dispatch.cu:156-218): expert-major slots, ascending token
    order inside an expert. -> [dispatched bf16 [S,H], token_map int32 [S],
    dispatched_weights fp32 [S]] with S = T * top_k."""
    op = "moe_dispatch"
    _cuda_contig(input, "input", op)
    _dtype(input, torch.bfloat16, "input", op)
    _req(input.dim() == 2, f"{op}: input must be a 2-D tensor [num_tokens, hidden_size].")
    _cuda_contig(topk_indices, "topk_indices", op)
    _dtype(topk_indices, torch.int32, "topk_indices", op)
    _req(topk_indices.dim() == 2, f"{op}: topk_indices must be a 2-D tensor [num_tokens, top_k].")
    _cuda_contig(topk_weights, "topk_weights", op)
    _dtype(topk_weights, torch.float32, "topk_weights", op)
    _req(topk_weights.dim() == 2, f"{op}: topk_weights must be a 2-D tensor [num_tokens, top_k].")
    _cuda_contig(expert_offsets, "expert_offsets", op)
    _dtype(expert_offsets, torch.int32, "expert_offsets", op)
    _req(expert_offsets.dim() == 1, f"{op}: expert_offsets must be a 1-D tensor [num_experts + 1].")
    T, H = input.shape
    K = topk_indices.shape[1]
    E = expert_offsets.shape[0] - 1
    _req(topk_indices.shape[0] == T and tuple(topk_weights.shape) == (T, K),
         f"{op}: topk_indices/topk_weights must be [num_tokens, top_k].")
    _req(H % 8 == 0, "hidden_size must be divisible by 8 for 128-bit vectorized access.")
    _req(1 <= E <= MAX_EXPERTS, f"{op}: num_experts must be in [1, 64].")
    _req(1 <= K <= MAX_TOP_K, f"{op}: top_k must be in [1, 6].")
    dev = input.device
    S = T * K
    dispatched = torch.empty((S, H), dtype=torch.bfloat16, device=dev)
    token_map = torch.empty((S,), dtype=torch.int32, device=dev)
    dw = torch.empty((S,), dtype=torch.float32, device=dev)
    ws = _ws(lib.dsk_moe_dispatch_workspace_size(T, E, K), dev)
    with torch.cuda.device(dev):
        check(lib.dsk_moe_dispatch(input.data_ptr(), H, topk_indices.data_ptr(),
                                   topk_weights.data_ptr(), expert_offsets.data_ptr(),
                                   dispatched.data_ptr(), token_map.data_ptr(), dw.data_ptr(),
                                   T, H, E, K, ws.data_ptr(), ws.numel(), stream_handle(dev)), op)
    return [dispatched, token_map, dw]


def moe_combine(expert_output: torch.Tensor, token_map: torch.Tensor,
                dispatched_weights: torch.Tensor, num_tokens: int) -> torch.Tensor:
    """Deterministic weighted combine (combine.cu:107-176): for every token, the
    slots that map to it are summed in ascending slot order in fp32 and rounded
    to bf16 once. No float atomics."""
    op = "moe_combine"
    _cuda_contig(expert_output, "expert_output", op)
    _dtype(expert_output, torch.bfloat16, "expert_output", op)
    _req(expert_output.dim() == 2, f"{op}: expert_output must be a 2-D tensor [total_slots, hidden_size].")
    _cuda_contig(token_map, "token_map", op)
    _dtype(token_map, torch.int32, "token_map", op)
    _req(token_map.dim() == 1, f"{op}: token_map must be a 1-D tensor [total_slots].")
    _cuda_contig(dispatched_weights, "dispatched_weights", op)
    _dtype(dispatched_weights, torch.float32, "dispatched_weights", op)
    _req(dispatched_weights.dim() == 1, f"{op}: dispatched_weights must be a 1-D tensor [total_slots].")
    S, H = expert_output.shape
    _req(token_map.shape[0] == S and dispatched_weights.shape[0] == S,
         f"{op}: token_map/dispatched_weights must have total_slots entries.")
    _req(int(num_tokens) > 0, "num_tokens must be positive.")
    _req(H % 8 == 0, f"{op}: hidden_size must be divisible by 8.")
    dev = expert_output.device
    out = torch.empty((int(num_tokens), H), dtype=torch.bfloat16, device=dev)
    ws = _ws(lib.dsk_moe_combine_workspace_size(S, int(num_tokens)), dev)
    with torch.cuda.device(dev):
        check(lib.dsk_moe_combine(expert_output.data_ptr(), token_map.data_ptr(),
                                  dispatched_weights.data_ptr(), out.data_ptr(), S,
                                  int(num_tokens), H, ws.data_ptr(), ws.numel(),
                                  stream_handle(dev)), op)
    return out


def swiglu(input: torch.Tensor) -> torch.Tensor:
    """silu(input[:, :I]) * input[:, I:] (swiglu.cu:142-170)."""
    op = "swiglu"
    _req(input.is_cuda, f"{op}: input must be a CUDA tensor.")
    _req(input.is_contiguous(), f"{op}: input must be contiguous.")
    _req(input.dtype == torch.bfloat16, f"{op}: input must be bfloat16.")
    _req(input.dim() == 2, f"{op}: input must be 2-D [total_tokens, 2*intermediate_size].")
    _req(input.shape[1] % 2 == 0, f"{op}: input inner dimension must be even.")
    rows, n2 = input.shape
    I = n2 // 2
    out = torch.empty((rows, I), dtype=torch.bfloat16, device=input.device)
    with torch.cuda.device(input.device):
        check(lib.dsk_swiglu(input.data_ptr(), out.data_ptr(), rows, I,
                             stream_handle(input.device)), op)
    return out


def _gemm_checks(op: str, a: torch.Tensor, aname: str, w: torch.Tensor, wname: str,
                 offsets: torch.Tensor) -> None:
    _req(a.is_cuda and a.is_contiguous(), f"{op}: {aname} must be a contiguous CUDA tensor.")
    _req(a.dtype == torch.bfloat16, f"{op}: {aname} must be bfloat16.")
    _req(a.dim() == 2, f"{op}: {aname} must be 2-D.")
    _req(w.is_cuda and w.is_contiguous(), f"{op}: {wname} must be a contiguous CUDA tensor.")
    _req(w.dtype == torch.bfloat16, f"{op}: {wname} must be bfloat16.")
    _req(w.dim() == 3, f"{op}: {wname} must be 3-D [num_experts, out, in].")
    _req(offsets.is_cuda and offsets.is_contiguous(),
         f"{op}: expert_offsets must be a contiguous CUDA tensor.")
    _req(offsets.dtype == torch.int32, f"{op}: expert_offsets must be int32.")
    _req(offsets.dim() == 1, f"{op}: expert_offsets must be 1-D [num_experts + 1].")
    _req(w.shape[2] == a.shape[1], f"{op}: {wname} inner dim does not match {aname}.")
    _req(offsets.shape[0] == w.shape[0] + 1, f"{op}: expert_offsets size must be num_experts + 1.")


def moe_gemm1(dispatched: torch.Tensor, packed_w1: torch.Tensor,
              expert_offsets: torch.Tensor) -> torch.Tensor:
    """Grouped gate|up projection (gemm1.cu:167-227): out[s] = dispatched[s] @
    packed_w1[e]^T for s in expert e's offset range; uncovered rows are zero."""
    op = "gemm1"
    _gemm_checks(op, dispatched, "dispatched", packed_w1, "packed_w1", expert_offsets)
    S, H = dispatched.shape
    E, N, _ = packed_w1.shape
    out = torch.empty((S, N), dtype=torch.bfloat16, device=dispatched.device)
    if S == 0:
        return out
    with torch.cuda.device(dispatched.device):
        check(lib.dsk_moe_gemm1(dispatched.data_ptr(), packed_w1.data_ptr(), out.data_ptr(),
                                expert_offsets.data_ptr(), S, E, H, N,
                                stream_handle(dispatched.device)), op)
    return out


def moe_gemm1_swiglu(dispatched: torch.Tensor, packed_w1: torch.Tensor,
                     expert_offsets: torch.Tensor) -> torch.Tensor:
    """moe_gemm1 followed by swiglu, fused: SwiGLU is applied to the fp32
    accumulators in the GEMM epilogue. -> [S, I] bf16."""
    op = "gemm1_swiglu"
    _gemm_checks(op, dispatched, "dispatched", packed_w1, "packed_w1", expert_offsets)
    S, H = dispatched.shape
    E, N, _ = packed_w1.shape
    _req(N % 2 == 0, f"{op}: packed_w1 rows must be 2*intermediate.")
    I = N // 2
    out = torch.empty((S, I), dtype=torch.bfloat16, device=dispatched.device)
    if S == 0:
        return out
    with torch.cuda.device(dispatched.device):
        check(lib.dsk_moe_gemm1_swiglu(dispatched.data_ptr(), packed_w1.data_ptr(),
                                       out.data_ptr(), expert_offsets.data_ptr(), S, E, H, I,
                                       stream_handle(dispatched.device)), op)
    return out


def moe_gemm2(swiglu_out: torch.Tensor, w2: torch.Tensor,
              expert_offsets: torch.Tensor) -> torch.Tensor:
    """Grouped down projection (gemm2.cu:136-195)."""
    op = "gemm2"
    _gemm_checks(op, swiglu_out, "swiglu_out", w2, "w2", expert_offsets)
    S, I = swiglu_out.shape
    E, H, _ = w2.shape
    out = torch.empty((S, H), dtype=torch.bfloat16, device=swiglu_out.device)
    if S == 0:
        return out
    with torch.cuda.device(swiglu_out.device):
        check(lib.dsk_moe_gemm2(swiglu_out.data_ptr(), w2.data_ptr(), out.data_ptr(),
                                expert_offsets.data_ptr(), S, E, I, H,
                                stream_handle(swiglu_out.device)), op)
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """x[..., K] @ weight[N, K]^T with the MFMA GEMM (bf16 in/out, fp32 acc).
    x may be a row-strided view (last dim contiguous, row stride % 8 == 0).
    weight is [N, K] row-major, or fragment-tiled [N/32, K/16, 64, 8]
    (tile_weights(w[None])[0]), which runs the weight-streaming kernel.
    out: optional [M, N] bf16 destination with a contiguous last dim and any row
    stride (e.g. rows of a cache); returned as given."""
    op = "linear"
    _req(x.is_cuda and weight.is_cuda, f"{op}: tensors must be CUDA tensors.")
    _req(x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16, f"{op}: bfloat16 only.")
    _req(weight.is_contiguous(), f"{op}: weight must be contiguous.")
    K = x.shape[-1]
    tiled = weight.dim() == 4
    if tiled:
        _req(tuple(weight.shape[2:]) == (64, 8) and weight.shape[1] * 16 == K,
             f"{op}: tiled weight must be [N/32, {K // 16}, 64, 8].")
        N = weight.shape[0] * 32
    else:
        _req(weight.dim() == 2, f"{op}: weight must be 2-D [N, K] or tiled 4-D.")
        N = weight.shape[0]
        _req(weight.shape[1] == K, f"{op}: weight inner dim {weight.shape[1]} != {K}.")
    x2 = x.reshape(-1, K) if not x.is_contiguous() or x.dim() != 2 else x
    _req(x2.stride(-1) == 1, f"{op}: last dim of x must be contiguous.")
    M = x2.shape[0]
    given = out is not None
    if given:
        _req(out.is_cuda and out.dtype == torch.bfloat16 and out.dim() == 2 and
             tuple(out.shape) == (M, N) and out.stride(1) == 1,
             f"{op}: out must be bf16 [{M}, {N}] with a contiguous last dim.")
    else:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if M:
        with torch.cuda.device(x.device):
            check(lib.dsk_linear_ex(x2.data_ptr(), x2.stride(0), weight.data_ptr(),
                                    1 if tiled else 0, out.data_ptr(), out.stride(0), M, K, N,
                                    stream_handle(x.device)), op)
    return out if given else out.view(*x.shape[:-1], N)


def _rowstat_operands(op: str, x: torch.Tensor, weight: torch.Tensor):
    _req(x.is_cuda and weight.is_cuda, f"{op}: tensors must be CUDA tensors.")
    _req(x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16, f"{op}: bfloat16 only.")
    K = x.shape[-1]
    _req(weight.is_contiguous() and weight.dim() == 4 and tuple(weight.shape[2:]) == (64, 8)
         and weight.shape[1] * 16 == K, f"{op}: weight must be fragment-tiled [N/32, {K // 16}, 64, 8].")
    x2 = x.reshape(-1, K)
    _req(x2.stride(-1) == 1, f"{op}: last dim of x must be contiguous.")
    return x2, K, weight.shape[0] * 32


def linear_rowsq(x: torch.Tensor, weight: torch.Tensor, col_begin: int, col_end: int):
    """(x @ weight^T, row_sumsq): the projection (tiled weight) and, per output
    row, the sum of squares of its bf16 outputs in columns [col_begin, col_end),
    as fp32 partials [(col_end - col_begin) / 256, rows] (one per 256 columns)."""
    op = "linear_rowsq"
    x2, K, N = _rowstat_operands(op, x, weight)
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _req(col_begin % 256 == 0 and col_end % 256 == 0 and 0 <= col_begin < col_end <= N,
         f"{op}: the column range must be 256-aligned inside [0, {N}).")
    ss = torch.empty(((col_end - col_begin) // 256, M), dtype=torch.float32, device=x.device)
    if M:
        with torch.cuda.device(x.device):
            check(lib.dsk_linear_rowsq(x2.data_ptr(), x2.stride(0), weight.data_ptr(),
                                       out.data_ptr(), N, M, K, N, ss.data_ptr(), M, col_begin,
                                       col_end, stream_handle(x.device)), op)
    return out.view(*x.shape[:-1], N), ss


def linear_rowscale(x: torch.Tensor, weight: torch.Tensor, row_sumsq: torch.Tensor,
                    n_cols: int, eps: float = 1e-6) -> torch.Tensor:
    """rsqrt(row_sumsq.sum(0) / n_cols + eps)[:, None] * (x @ weight^T): an RMS
    norm of x's rows (statistics from linear_rowsq) applied in the epilogue of
    the projection whose weight carries the norm weight per input column."""
    op = "linear_rowscale"
    x2, K, N = _rowstat_operands(op, x, weight)
    M = x2.shape[0]
    _req(row_sumsq.is_cuda and row_sumsq.dtype == torch.float32 and row_sumsq.dim() == 2
         and row_sumsq.shape[1] == M and row_sumsq.is_contiguous(),
         f"{op}: row_sumsq must be a contiguous float32 [parts, {M}] CUDA tensor.")
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if M:
        with torch.cuda.device(x.device):
            check(lib.dsk_linear_rowscale(x2.data_ptr(), x2.stride(0), weight.data_ptr(),
                                          out.data_ptr(), N, M, K, N, row_sumsq.data_ptr(), M,
                                          row_sumsq.shape[0], int(n_cols), float(eps),
                                          stream_handle(x.device)), op)
    return out.view(*x.shape[:-1], N)


def linear_split(x: torch.Tensor, weight: torch.Tensor, out0: torch.Tensor,
                 out1: torch.Tensor) -> None:
    """x[M, K] @ weight^T with columns [0, n0) written to out0 [M, n0] and the
    rest to out1 [M, N - n0] (dsk_linear_split): one launch for M <= 64. weight
    is fragment-tiled [N/32, K/16, 64, 8]; n0 = out0.shape[1] must be a multiple
    of 64. Both outputs may be row-strided views with a contiguous last dim (for
    example out1 = rows of a cache)."""
    op = "linear_split"
    _req(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1,
         f"{op}: x must be a bf16 CUDA tensor [M, K] with a contiguous last dim.")
    M, K = x.shape
    _req(weight.is_cuda and weight.is_contiguous() and weight.dtype == torch.bfloat16 and
         weight.dim() == 4 and tuple(weight.shape[2:]) == (64, 8) and weight.shape[1] * 16 == K,
         f"{op}: weight must be tiled [N/32, {K // 16}, 64, 8].")
    N = weight.shape[0] * 32
    for name, o in (("out0", out0), ("out1", out1)):
        _req(o.is_cuda and o.dtype == torch.bfloat16 and o.dim() == 2 and o.shape[0] == M and
             o.stride(1) == 1, f"{op}: {name} must be bf16 [{M}, n] with a contiguous last dim.")
    n0 = out0.shape[1]
    _req(n0 + out1.shape[1] == N, f"{op}: out0 and out1 widths must add up to {N}.")
    if M:
        with torch.cuda.device(x.device):
            check(lib.dsk_linear_split(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                       out0.data_ptr(), out0.stride(0), out1.data_ptr(),
                                       out1.stride(0), M, K, N, n0, stream_handle(x.device)), op)


def linear_batched(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """out[b] = x[b] @ weight[b]^T for every entry b of a batch, in one launch
    (dsk_linear_batched), up to 64 rows per entry. x: bf16 [batch, M, K], any
    strides with a contiguous last dim; weight: fragment-tiled [batch, N/32,
    K/16, 64, 8] (tile_weights of a [batch, N, K] stack); out: optional [batch,
    M, N] destination view. Returns out."""
    op = "linear_batched"
    _req(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3 and x.stride(2) == 1,
         f"{op}: x must be a bf16 CUDA tensor [batch, M, K] with a contiguous last dim.")
    nb, M, K = x.shape
    _req(weight.is_cuda and weight.is_contiguous() and weight.dtype == torch.bfloat16 and
         weight.dim() == 5 and weight.shape[0] == nb and tuple(weight.shape[3:]) == (64, 8) and
         weight.shape[2] * 16 == K, f"{op}: weight must be tiled [{nb}, N/32, {K // 16}, 64, 8].")
    N = weight.shape[1] * 32
    if out is None:
        out = torch.empty((nb, M, N), dtype=torch.bfloat16, device=x.device)
    _req(out.is_cuda and out.dtype == torch.bfloat16 and tuple(out.shape) == (nb, M, N) and
         out.stride(2) == 1, f"{op}: out must be bf16 [{nb}, {M}, {N}] with a contiguous last dim.")
    if nb and M:
        with torch.cuda.device(x.device):
            check(lib.dsk_linear_batched(x.data_ptr(), x.stride(1), x.stride(0), weight.data_ptr(),
                                         out.data_ptr(), out.stride(1), out.stride(0), nb, M, K,
                                         N, stream_handle(x.device)), op)
    return out


def linear_rows(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor = None,
                out1: torch.Tensor = None, n_split: int = None) -> torch.Tensor:
    """x @ weight^T for at most 4 token rows on the vector ALU (dsk_linear_rows),
    spread over N/8 lane groups: the projections of a one-token decode step.
    x: bf16 [M, K] or [batch, M, K] (contiguous last dim); weight: fragment-tiled
    [N/32, K/16, 64, 8] (shared by every batch entry) or [batch, N/32, K/16, 64,
    8]; out: optional destination
    view ([.., M, n_split] when out1 is given); out1 with n_split: columns
    n_split.. go to out1 ([.., M, N - n_split]). Returns out."""
    op = "linear_rows"
    batched = x.dim() == 3
    _req(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() in (2, 3) and x.stride(-1) == 1,
         f"{op}: x must be a bf16 CUDA tensor [M, K] or [batch, M, K] with a contiguous last dim.")
    xb = x if batched else x[None]
    nb, M, K = xb.shape
    wb = weight if weight.dim() == 5 else weight[None]
    _req(weight.is_cuda and weight.is_contiguous() and weight.dtype == torch.bfloat16 and
         wb.dim() == 5 and wb.shape[0] in (1, nb) and tuple(wb.shape[3:]) == (64, 8) and
         wb.shape[2] * 16 == K, f"{op}: weight must be tiled [N/32, {K // 16}, 64, 8] per entry.")
    N = wb.shape[1] * 32
    ns = N if out1 is None else n_split
    _req(ns is not None and 0 <= ns <= N, f"{op}: n_split must be in [0, N] with out1.")
    shape0 = (nb, M, ns) if batched else (M, ns)
    if out is None:
        out = torch.empty(shape0, dtype=torch.bfloat16, device=x.device)
    for t, shp, nm in ((out, shape0, "out"),) + (((out1, (nb, M, N - ns) if batched else
                                                  (M, N - ns), "out1"),) if out1 is not None else ()):
        _req(t.is_cuda and t.dtype == torch.bfloat16 and tuple(t.shape) == shp and t.stride(-1) == 1,
             f"{op}: {nm} must be bf16 {list(shp)} with a contiguous last dim.")
    o0 = out if batched else out[None]
    o1 = (out1 if batched else out1[None]) if out1 is not None else None
    if nb and M:
        with torch.cuda.device(x.device):
            check(lib.dsk_linear_rows(xb.data_ptr(), xb.stride(1), xb.stride(0), wb.data_ptr(),
                                      wb[0].numel() if wb.shape[0] > 1 else 0, o0.data_ptr(),
                                      o0.stride(1),
                                      o0.stride(0), o1.data_ptr() if o1 is not None else None,
                                      o1.stride(1) if o1 is not None else 0,
                                      o1.stride(0) if o1 is not None else 0, ns, nb, M, K, N,
                                      stream_handle(x.device)), op)
    return out


def kv_upproj(normed_kv: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """kv_b_proj up-projection (kv_upproj.cu:133-178): [..., 512] -> [..., out_dim].
    weight is [out_dim, kv_lora_rank] as in the reference, or its fragment-tiled
    form [out_dim/32, kv_lora_rank/16, 64, 8] (tile_weights(w[None])[0])."""
    op = "kv_upproj"
    _req(normed_kv.is_cuda and normed_kv.is_contiguous(),
         f"{op}: normed_kv must be a contiguous CUDA tensor.")
    _req(normed_kv.dtype == torch.bfloat16, f"{op}: normed_kv must be bfloat16.")
    _req(normed_kv.dim() >= 2, f"{op}: normed_kv must have at least 2 dimensions.")
    _req(weight.is_cuda and weight.is_contiguous(), f"{op}: weight must be a contiguous CUDA tensor.")
    _req(weight.dtype == torch.bfloat16, f"{op}: weight must be bfloat16.")
    r = normed_kv.shape[-1]
    tiled = weight.dim() == 4
    if tiled:
        _req(tuple(weight.shape[2:]) == (64, 8) and weight.shape[1] * 16 == r,
             f"{op}: tiled weight must be [out_dim/32, {r // 16}, 64, 8].")
        n = weight.shape[0] * 32
    else:
        _req(weight.dim() == 2, f"{op}: weight must be 2-D [out_dim, kv_lora_rank].")
        _req(weight.shape[1] == r,
             f"{op}: weight inner dim {weight.shape[1]} must match normed_kv last dim {r}.")
        n = weight.shape[0]
    rows = normed_kv.numel() // r
    out = torch.empty((*normed_kv.shape[:-1], n), dtype=torch.bfloat16, device=normed_kv.device)
    if rows:
        with torch.cuda.device(normed_kv.device):
            if tiled:
                check(lib.dsk_linear_ex(normed_kv.data_ptr(), r, weight.data_ptr(), 1,
                                        out.data_ptr(), n, rows, r, n,
                                        stream_handle(normed_kv.device)), op)
            else:
                check(lib.dsk_kv_upproj(normed_kv.data_ptr(), r, weight.data_ptr(),
                                        out.data_ptr(), rows, r, n,
                                        stream_handle(normed_kv.device)), op)
    return out


def rms_norm(input: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last dim (rms_norm.cu:158-192): bf16 input, fp32 weight,
    bf16 output. An fp32 input selects the fp32-in/fp32-out kernel. The input may
    be a row-strided view (last dim contiguous), e.g. the latent slice of kv_a."""
    op = "rms_norm"
    _req(input.is_cuda, f"{op}: input must be a CUDA tensor.")
    _req(weight.is_cuda, f"{op}: weight must be a CUDA tensor.")
    _req(input.dtype in (torch.bfloat16, torch.float32), f"{op}: input must be bfloat16.")
    _req(weight.dtype == torch.float32,
         f"{op}: weight must be float32 (default nn.Parameter dtype).")
    _req(input.dim() >= 2, f"{op}: input must have at least 2 dimensions.")
    H = input.shape[-1]
    _req(weight.numel() == H,
         f"{op}: weight size {weight.numel()} does not match input hidden_size {H}.")
    weight = weight.contiguous()
    if input.dtype == torch.bfloat16:
        _req(H % 2 == 0, f"{op}: hidden_size must be even for bfloat162 vectorisation.")
    # Flatten leading dims without a copy when the rows are uniformly strided.
    try:
        x2 = input.view(-1, H)
    except RuntimeError:
        x2 = None
    if x2 is None or x2.stride(-1) != 1:
        x2 = input.contiguous().view(-1, H)
    rows = x2.shape[0]
    out = torch.empty(input.shape, dtype=input.dtype, device=input.device)
    if rows == 0:
        return out
    fn = lib.dsk_rms_norm if input.dtype == torch.bfloat16 else lib.dsk_rms_norm_f32
    with torch.cuda.device(input.device):
        check(fn(x2.data_ptr(), x2.stride(0), weight.data_ptr(), out.data_ptr(), H, rows, H,
                 float(eps), stream_handle(input.device)), op)
    return out


def _rope_strides(t: torch.Tensor, name: str):
    _req(t.dim() == 4, f"rope: {name} must be 4-D.")
    _req(t.stride(3) == 1, f"rope: {name} last dim must be contiguous.")
    b, h, s, d = t.shape
    sb, sh, ss = t.stride(0), t.stride(1), t.stride(2)
    return sb, (sh if h > 1 else 0), ss


def attn_softmax_(scores: torch.Tensor, scale: float, causal: bool = True,
                  kv_len: int = None, mask: torch.Tensor = None) -> torch.Tensor:
    """In place over bf16 scores [..., q_len, L] (last dim contiguous, rows
    16-byte aligned): softmax_fp32(bf16(scores * scale) + mask) rounded to bf16,
    the eager sequence of DeepSeekMLA.forward (mla.py:366-381) in one pass.
    kv_len: the number of keys (default L); the columns kv_len.. up to the next
    multiple of 8 are written as 0, so a score buffer padded to 16-byte rows
    feeds P.V with exact zeros. causal: query i sees keys j <= i + kv_len - q_len.
    mask: an additive attention_mask (bf16 or fp32, -inf where masked)
    broadcastable to [b, h, q_len, kv_len] for 4-D scores [b, h, q_len, L]
    (mla.py:374: `attn_weights + attention_mask`, in the dtype torch promotes
    the sum to), applied in place of the causal mask when causal is False.
    Returns scores."""
    op = "attn_softmax"
    _req(scores.is_cuda, f"{op}: scores must be a CUDA tensor.")
    _dtype(scores, torch.bfloat16, "scores", op)
    _req(scores.dim() >= 2 and scores.stride(-1) == 1, f"{op}: last dim must be contiguous.")
    q_len, L = scores.shape[-2], scores.shape[-1]
    kv_len = L if kv_len is None else int(kv_len)
    _req(0 < kv_len <= L and (kv_len + 7) // 8 * 8 <= L,
         f"{op}: kv_len {kv_len} must be in 1..{L} with room for its 8-key padding.")
    flat = scores.view(-1, L) if scores.is_contiguous() else None
    _req(flat is not None, f"{op}: scores must be contiguous.")
    rows = flat.shape[0]
    if not rows:
        return scores
    st = stream_handle(scores.device)
    if mask is None:
        with torch.cuda.device(scores.device):
            check(lib.dsk_attn_softmax(flat.data_ptr(), L, rows, kv_len, q_len, float(scale),
                                       1 if causal else 0, st), op)
        return scores
    _req(scores.dim() == 4, f"{op}: a mask needs 4-D scores [b, h, q_len, L].")
    _req(mask.is_cuda and mask.device == scores.device, f"{op}: mask must be on the scores' device.")
    _req(mask.dtype in (torch.bfloat16, torch.float32), f"{op}: mask must be bf16 or fp32.")
    b, h = scores.shape[0], scores.shape[1]
    _req(mask.dim() <= 4, f"{op}: mask must have at most 4 dims.")
    m = mask.reshape((1,) * (4 - mask.dim()) + tuple(mask.shape))
    try:
        m = m.expand(b, h, q_len, kv_len)
    except RuntimeError:
        raise RuntimeError(f"{op}: mask {tuple(mask.shape)} does not broadcast to "
                           f"[{b}, {h}, {q_len}, {kv_len}].") from None
    if m.stride(-1) != 1:
        m = m.contiguous()
    with torch.cuda.device(scores.device):
        check(lib.dsk_attn_softmax_masked(
            flat.data_ptr(), L, rows, kv_len, q_len, h, float(scale), 1 if causal else 0,
            m.data_ptr(), 1 if m.dtype == torch.float32 else 0, m.stride(0), m.stride(1),
            m.stride(2), st), op)
    return scores


def mla_attn_pack(q: torch.Tensor, kv: torch.Tensor, k_pe: torch.Tensor, cos: torch.Tensor,
                  sin: torch.Tensor, heads: int = 16, pad: bool = False):
    """The head-major operands of DeepSeekMLA.forward's attention (mla.py:354-366)
    in one pass: Q = (q_nope | rope(q_pe)) [b, h, s, 192], K^T = (k_nope |
    rope(k_pe) for every head)^T [b, h, 192, s] and V [b, h, s, 128], all
    contiguous. q: bf16 [b, s, h*192] (q_proj output, each head nope then rope
    part), kv: bf16 [b, s, h*256] (kv_b_proj output, each head k_nope then v),
    k_pe: bf16 [b, s, 64] (raw shared RoPE key); each may be a view with strided
    rows and a contiguous last dim. cos/sin: [>= s, 64] tables by position, or
    [b, >= s, 64] per batch entry (the tables indexed by position_ids), cast to
    bf16 as the RoPE op uses them.
    pad: K^T and V get sp = s rounded up to 8 positions ([b, h, 192, sp],
    [b, h, sp, 128]) with zero padding, so that s need not be a multiple of 8;
    without it s must be."""
    op = "mla_attn_pack"
    for t, nm in ((q, "q"), (kv, "kv"), (k_pe, "k_pe"), (cos, "cos"), (sin, "sin")):
        _req(isinstance(t, torch.Tensor) and t.is_cuda, f"{op}: {nm} must be a CUDA tensor.")
    for t, nm in ((q, "q"), (kv, "kv"), (k_pe, "k_pe")):
        _dtype(t, torch.bfloat16, nm, op)
        _req(t.dim() == 3 and t.stride(2) == 1, f"{op}: {nm} must be 3-D with a contiguous last dim.")
    b, s, nq = q.shape
    _req(nq == heads * 192 and kv.shape == (b, s, heads * 256) and k_pe.shape == (b, s, 64),
         f"{op}: expected q [b, s, {heads}*192], kv [b, s, {heads}*256], k_pe [b, s, 64].")
    for t, nm in ((q, "q"), (kv, "kv"), (k_pe, "k_pe")):
        _req(b <= 1 or t.stride(0) == s * t.stride(1),
             f"{op}: {nm} rows must be evenly spaced over batch and sequence.")
    _req(pad or s % 8 == 0, f"{op}: s must be a multiple of 8 (or pass pad=True).")
    cb = cos.to(torch.bfloat16).contiguous()
    sb = sin.to(torch.bfloat16).contiguous()
    _req(sb.shape == cb.shape and cb.dim() in (2, 3) and cb.shape[-2] >= s and cb.shape[-1] == 64
         and (cb.dim() == 2 or cb.shape[0] == b),
         f"{op}: cos/sin must be [>= s, 64] or [b, >= s, 64].")
    sp = (s + 7) // 8 * 8 if pad else s
    dev = q.device
    q_out = torch.empty((b, heads, s, 192), dtype=torch.bfloat16, device=dev)
    k_t = torch.empty((b, heads, 192, sp), dtype=torch.bfloat16, device=dev)
    v = torch.empty((b, heads, sp, 128), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        check(lib.dsk_mla_attn_pack_ex(q.data_ptr(), q.stride(1), kv.data_ptr(), kv.stride(1),
                                       k_pe.data_ptr(), k_pe.stride(1), cb.data_ptr(),
                                       sb.data_ptr(), cb.stride(-2),
                                       cb.stride(0) if cb.dim() == 3 else 0, q_out.data_ptr(),
                                       k_t.data_ptr(), v.data_ptr(), b, s, sp, heads, 128, 64,
                                       128, stream_handle(dev)), op)
    return q_out, k_t, v


def _rows_overlap(a: torch.Tensor, wa: int, b: torch.Tensor, wb: int) -> bool:
    """Whether views a and b ([bsz, L, w] with the same batch and token strides)
    share an element: separate storages never do; inside one buffer, b's column
    offset within a's token row decides."""
    if a.untyped_storage().data_ptr() != b.untyped_storage().data_ptr():
        return False
    ld, lb = a.stride(1), a.stride(0)
    B, L = a.shape[0], a.shape[1]
    span = (B - 1) * lb + (L - 1) * ld
    d = b.storage_offset() - a.storage_offset()
    if d >= span + wa or -d >= span + wb:
        return False
    if B > 1 and lb % ld != 0:
        return True
    c = d % ld
    return c < wa or c + wb > ld


def mla_decode_attention(q_abs: torch.Tensor, q_pe: torch.Tensor, latent: torch.Tensor,
                         k_pe: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, scale: float,
                         eps: float = 1e-6, out: torch.Tensor = None,
                         k_rope: torch.Tensor = None, rope_len: int = 0) -> torch.Tensor:
    """Absorbed MLA attention of T = bsz * n new tokens over the raw latent
    cache (the attention of mla.py:356-384 on cached tokens, latent RMSNorm
    applied on the fly).
    q_abs: bf16 [T, 16, 512] ((W_UK * w)^T q_nope per head); q_pe: bf16
    [T, 16, 64], raw (pre-RoPE); latent / k_pe: bf16 [bsz, L, 512] / [bsz, L, 64]
    cache views sharing their batch and token strides, the last n tokens being
    the new ones; cos/sin: bf16 [>= L, 64] by position. k_rope: bf16
    [bsz, L, 64] with the same strides, the keys after RoPE: rows < rope_len
    are read, rows from rope_len on are rotated from k_pe and written (None: a
    scratch buffer, every key rotated here). All may be strided views with a
    contiguous last dim; k_rope must not overlap latent or k_pe. Without k_rope
    the op allocates a scratch of the latent's strides (up to bsz x token
    stride x L elements, of which it writes 64 per token) and rotates all L
    keys on every call; LatentKVCache.k_rope keeps them across calls instead.
    Returns bf16 [T, 16, 512] (into `out` if given): sum_j softmax_j r_j x_j
    per head."""
    op = "mla_decode_attention"
    for t, nm in ((q_abs, "q_abs"), (q_pe, "q_pe"), (latent, "latent"), (k_pe, "k_pe"),
                  (cos, "cos"), (sin, "sin")):
        _req(isinstance(t, torch.Tensor) and t.is_cuda, f"{op}: {nm} must be a CUDA tensor.")
        _dtype(t, torch.bfloat16, nm, op)
        _req(t.stride(-1) == 1, f"{op}: {nm} last dim must be contiguous.")
    _req(q_abs.dim() == 3 and q_abs.shape[1:] == (16, 512), f"{op}: q_abs must be [T, 16, 512].")
    T = q_abs.shape[0]
    _req(q_pe.shape == (T, 16, 64), f"{op}: q_pe must be [T, 16, 64].")
    _req(latent.dim() == 3 and latent.shape[2] == 512, f"{op}: latent must be [bsz, L, 512].")
    b, L = latent.shape[0], latent.shape[1]
    _req(k_pe.shape == (b, L, 64), f"{op}: k_pe must be [bsz, L, 64].")
    _req(latent.stride()[:2] == k_pe.stride()[:2],
         f"{op}: latent and k_pe must share batch and token strides.")
    if k_rope is None:
        # scratch for the rotated keys with the latent's strides (the kernel
        # addresses all three by one token stride); only its 64 columns per
        # token are written, every key rotated here (rope_len 0)
        sb, st_ = latent.stride(0), latent.stride(1)
        extent = (b - 1) * sb + (L - 1) * st_ + 64
        k_rope = torch.empty(extent, dtype=torch.bfloat16,
                             device=latent.device).as_strided((b, L, 64), (sb, st_, 1))
        rope_len = 0
    _req(isinstance(k_rope, torch.Tensor) and k_rope.is_cuda and k_rope.dtype == torch.bfloat16
         and k_rope.shape == (b, L, 64) and k_rope.stride()[:2] == latent.stride()[:2]
         and k_rope.stride(-1) == 1,
         f"{op}: k_rope must be bf16 [bsz, L, 64] with the strides of latent.")
    for t, nm, w in ((latent, "latent", 512), (k_pe, "k_pe", 64)):
        _req(not _rows_overlap(k_rope, 64, t, w),
             f"{op}: k_rope overlaps {nm} (it is written while {nm} is read).")
    _req(isinstance(rope_len, int) and 0 <= rope_len <= L, f"{op}: need 0 <= rope_len <= {L}.")
    _req(b > 0 and T % b == 0, f"{op}: T={T} is not a multiple of bsz={b}.")
    n = T // b
    _req(n <= L, f"{op}: {n} new tokens but only {L} in the cache.")
    _req(cos.shape == sin.shape and cos.dim() == 2 and cos.shape[1] == 64 and cos.shape[0] >= L,
         f"{op}: cos/sin must be [>= {L}, 64].")
    cos, sin = cos.contiguous(), sin.contiguous()
    if out is None:
        out = torch.empty((T, 16, 512), dtype=torch.bfloat16, device=q_abs.device)
    _req(out.shape == (T, 16, 512) and out.dtype == torch.bfloat16 and out.stride(-1) == 1,
         f"{op}: out must be bf16 [T, 16, 512] with a contiguous last dim.")
    if T == 0:
        return out
    ws = _ws(lib.dsk_mla_decode_workspace_size(b, n, L), q_abs.device)
    ld_batch = latent.stride(0) if b > 1 else L * latent.stride(1)
    with torch.cuda.device(q_abs.device):
        check(lib.dsk_mla_decode_attention(
            q_abs.data_ptr(), q_abs.stride(0), q_abs.stride(1), q_pe.data_ptr(), q_pe.stride(0),
            q_pe.stride(1), latent.data_ptr(), k_pe.data_ptr(), k_rope.data_ptr(), rope_len,
            latent.stride(1), ld_batch, cos.data_ptr(), sin.data_ptr(), float(eps), float(scale),
            b, n, L, out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(),
            stream_handle(q_abs.device)), op)
    return out


def rope_single(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The RoPE of `rope` on one tensor x [b, h, s, d] (a strided view with a
    contiguous last dim) with the pre-indexed cos/sin [b, 1, s, d]; returns a
    contiguous [b, h, s, d]."""
    op = "rope"
    for t in (x, cos, sin):
        _req(t.is_cuda and t.dtype == torch.bfloat16, f"{op}: inputs must be bf16 CUDA tensors.")
        _req(t.dim() == 4, f"{op}: inputs must be 4-D.")
    b, h, s, d = x.shape
    _req(cos.shape == (b, 1, s, d) and sin.shape == (b, 1, s, d), f"{op}: cos/sin shape incompatible.")
    if cos.stride(3) != 1 or sin.stride(3) != 1 or cos.stride() != sin.stride():
        cos, sin = cos.contiguous(), sin.contiguous()
    sb, sh, ss = _rope_strides(x, "x")
    out = torch.empty((b, h, s, d), dtype=torch.bfloat16, device=x.device)
    with torch.cuda.device(x.device):
        check(lib.dsk_rope(x.data_ptr(), sb, sh, ss, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                           cos.stride(2), out.data_ptr(), b, h, s, d,
                           stream_handle(x.device)), op)
    return out


def rope(q_pe: torch.Tensor, k_pe: torch.Tensor, cos: torch.Tensor,
         sin: torch.Tensor) -> List[torch.Tensor]:
    """Interleaved -> half RoPE on q_pe [b,h,s,d] and k_pe [b,1,s,d] with the
    pre-indexed cos/sin [b,1,s,d] (rope.cu:139-207). Inputs may be strided
    views (last dim contiguous); outputs are contiguous."""
    op = "rope"
    for t, n in ((q_pe, "q_pe"), (k_pe, "k_pe"), (cos, "cos"), (sin, "sin")):
        _req(t.is_cuda, f"{op}: all inputs must be CUDA tensors.")
        _req(t.dtype == torch.bfloat16, f"{op}: all inputs must be bfloat16.")
    _req(q_pe.dim() == 4, f"{op}: q_pe must be 4-D [bsz, heads, seq, rope_dim].")
    _req(k_pe.dim() == 4, f"{op}: k_pe must be 4-D [bsz, 1, seq, rope_dim].")
    _req(cos.dim() == 4, f"{op}: cos must be 4-D [bsz, 1, seq, rope_dim].")
    _req(sin.dim() == 4, f"{op}: sin must be 4-D [bsz, 1, seq, rope_dim].")
    b, hq, s, d = q_pe.shape
    _req(k_pe.shape[0] == b and k_pe.shape[2] == s and k_pe.shape[3] == d,
         f"{op}: k_pe shape {list(k_pe.shape)} incompatible with q_pe.")
    _req(cos.shape[0] == b and cos.shape[2] == s and cos.shape[3] == d,
         f"{op}: cos shape incompatible.")
    _req(sin.shape[0] == b and sin.shape[2] == s and sin.shape[3] == d,
         f"{op}: sin shape incompatible.")
    _req(d % 2 == 0, f"{op}: rope_dim must be even.")
    _req(d % 8 == 0, f"{op}: rope_dim must be a multiple of 8.")
    if cos.stride(3) != 1 or sin.stride(3) != 1 or cos.stride() != sin.stride():
        cos, sin = cos.contiguous(), sin.contiguous()
    cb, cs = cos.stride(0), cos.stride(2)
    qsb, qsh, qss = _rope_strides(q_pe, "q_pe")
    ksb, ksh, kss = _rope_strides(k_pe, "k_pe")
    hk = k_pe.shape[1]
    q_rot = torch.empty((b, hq, s, d), dtype=torch.bfloat16, device=q_pe.device)
    k_rot = torch.empty((b, hk, s, d), dtype=torch.bfloat16, device=q_pe.device)
    with torch.cuda.device(q_pe.device):
        check(lib.dsk_rope_qk(q_pe.data_ptr(), qsb, qsh, qss, k_pe.data_ptr(), ksb, ksh, kss,
                              cos.data_ptr(), sin.data_ptr(), cb, cs, q_rot.data_ptr(),
                              k_rot.data_ptr(), b, hq, hk, s, d,
                              stream_handle(q_pe.device)), op)
    return [q_rot, k_rot]
