"""CPU oracle of the batch-1 int8 decode path: TEST INFRASTRUCTURE ONLY.

A restatement, on the CPU, of the reference's arithmetic for this path. It exists
to check the HIP kernels and to time a CPU baseline. Only tests/, the smoke check
in __graft_entry__.py and the cpu_baseline leg of bench.py may import it; the
product (efficientgpt_amd) never does and has no CPU fallback.

Modules and what pins each function (checks live in tests/test_oracle.py):
  numerics      bf16 round-to-nearest-even on float32 arrays.
                Pinned: hand-computed bit patterns, ties to even, NaN/Inf, and
                agreement with torch's own float32->bfloat16 cast.
  int8          quantize_weight, the decode / prefill / naive int8 linear formulas,
                fp64 truth, the reference's tolerance rules.
                Pinned: known-answer quantisation (half-even ties), the closed-form
                invariants of research/realmodel/test_int8_linear.py:43-53, brute-force
                loops on tiny shapes, and planted mistakes (no scale, dropped last K
                block, unsigned bytes) that the tolerance rule must reject.
  attention     fp64 masked GQA decode attention, fp64 causal prompt-block
                attention, and an fp32 restatement of the reference's split-K + combine.
                Pinned: position 0 returns v[0], constant keys give the mean of v,
                Hkv == Hq equals the multi-head form, GQA equals repeat_kv + MHA,
                agreement with torch's scaled_dot_product_attention in float64, and a
                planted off-by-one mask that must be caught; the prompt block row by
                row equals the decode form at position pos0 + t and torch's causal
                SDPA (is_causal) in float64, and a mask shifted by one is caught.
  qwen3         Qwen3 decoder step (RMSNorm, q/k-norm, RoPE, GQA attention, SwiGLU,
                int8 linears by the reference's row rule) in torch on the CPU.
                Pinned: logits and greedy tokens of transformers' own
                Qwen3ForCausalLM (a third-party library, installed here) on tiny
                configurations, bf16 and fp32.
"""
