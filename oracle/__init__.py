"""CPU oracle for the flat-cost speculative-verify path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's arithmetic on this path, used to check the device path:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import it, and never
as the thing measured or shipped. The product (skinny_mlx) never imports this package.

Modules and the reference code each restates:
  w4.py      MLX affine W4 g64 format, dequant + matmul (skinny_mlx/qmm.py:8-9, 96-115,
             132-152; patch.py:30-35, 80-81), bf16 rounding, the fragment relayout.
  gdn.py     gated delta rule recurrence and the GDN mixer around it (bench/reversal_check.py:
             21-25, 43-47; third-party mlx_lm gated_delta_update, cross-checked against
             transformers' qwen3_5 restatement), conv window and state selection for
             rollback (skinny_mlx/rollback.py:58-73).
  accept.py  greedy acceptance: row argmax with first-index ties, longest matching prefix,
             bonus token (skinny_mlx/spec.py:137-147); prompt-lookup drafting (spec.py:32-51).
  model.py   the decoder forward (dense and hybrid) used by the end-to-end parity tests
             (skinny_mlx/spec.py:24-29; mtp.py:51-67).

How each function is pinned (golden vectors, closed forms, brute force) is listed in the
module docstrings; see tests/test_oracle_*.py.
"""
