"""CPU oracle for the DeepSeek-V2-Lite MoE layer and MLA helper kernels.

TEST INFRASTRUCTURE ONLY. This package restates the reference algorithms
(sahan974/DeepSeek-V2-Lite-CUDA, src/reference/*.py and the kernel formulas in
src/kernels/**) in numpy, each function citing the file:line it follows. It is
the checker for the HIP path: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it, and never as the thing measured or
shipped. The product (deepseek-v2-lite-cuda_amd/ds_kernels) never imports it.

How each function is pinned (tests/test_oracle_*.py):
  moe.route            torch.topk on torch.softmax (library) on tie-free inputs,
                       all-zero-logits KAT (reference test_moe_routing_kernel.py:155-173,
                       with ties to the lower index), partial-tie case, brute force.
  moe.scan             reference scan KATs (test_moe_scan_kernel.py:64-164).
  moe.permute/dispatch brute-force O(S^2) definition on tiny inputs + the
                       reference dispatch test's invariants (test_moe_dispatch_kernel.py:114-210).
  moe.grouped_linear   torch.nn.functional.linear per expert (library).
  moe.swiglu           torch.nn.functional.silu (library).
  moe.combine          pure-Python loop (test_moe_combine_kernel.py:47-64), zero-weight KAT.
  moe.moe_layer        dense formulation through torch (every expert on every token,
                       masked by the routing weights), a differently structured computation.
  mla.rms_norm         torch.nn.functional.rms_norm (library).
  mla.yarn_inv_freq    closed forms of the pure-extrapolation / pure-interpolation
                       bands and the correction range (10, 23) for dim 64.
  mla.rope             complex multiplication (x_2k + i x_2k+1) * e^{i theta}.
  mla.mla_forward /    composition of the pinned parts; attention core checked against
  mla.decoder_layer    torch.nn.functional.scaled_dot_product_attention (fp32, CPU).
"""
