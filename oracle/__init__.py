"""CPU oracle for the Qwen3 decode hot path — TEST INFRASTRUCTURE ONLY.

Restatements of the reference's (ErnestW2019/acorninfer) algorithms, each
function citing the reference file:line it follows. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker or the timed CPU baseline; the product
package (acorninfer_amd) never imports it and has no CPU fallback.

Modules:
  ops_ref     K1 / K2 / K3 / RMSNorm / RoPE and block-table restatements (torch CPU)
  quant_ref   W8 / W4 quantise, pack, dequant, GEMM references (numpy)
  sampler_ref temperature -> top-k -> top-p processing and inverse-CDF draw
  qwen3_ref   Qwen3 dense model: SDPA prefill/decode path and greedy loop

How each function is pinned (golden vectors, known answers, closed forms,
invariants) is listed in the module docstrings and tested in
tests/test_oracle_*.py.
"""
