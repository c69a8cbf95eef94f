"""CPU oracle for the routed-MoE decode hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path
the MI355X library accelerates.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg may import it, and only as the checker or
as the timed CPU baseline — never as the thing shipped or measured on the GPU.
The product path (``sluice_amd``) never imports this package.

Modules and what each follows:
  routing  top-k routing closed forms (vLLM select_experts as called at
           src/sluice/offloader.py:2583-2585; softmax greedy / softmax+renorm /
           sigmoid group-limited) with a specified tie rule.
  slru     the slot cache and gap state machine, line by line after
           src/sluice/offloader.py:121-169, 895-1044, 2009-2123, 2362-2467.
  moe      dense per-token SwiGLU expert product and weighted combine
           (vLLM fused_experts as called at src/sluice/offloader.py:2590-2599),
           plus fp8 e4m3fn 128x128 block dequantisation.

How each part is pinned (tests/test_oracle_*.py):
  routing  against transformers' DeepSeek-V2 / Qwen3-MoE / DeepSeek-V3 routers
           on tie-free logits, brute force over all k-subsets for tiny E, and
           the tie rule on constructed ties.
  slru     against fixtures written by running the reference's own
           ExpertStreamOffloader._router_split_gap in this container
           (tests/golden/make_slru_vectors.py), plus invariants and
           hand-worked traces.
  moe      against transformers' Qwen3MoeExperts / DeepseekV2Experts forward
           and closed-form cases (single expert, zero weights, unmapped
           experts contribute zero); fp8 decode against torch.float8_e4m3fn.
"""
