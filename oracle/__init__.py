"""CPU oracle for liteinfer's `paged` attention path — TEST INFRASTRUCTURE ONLY.

A from-scratch restatement, in numpy, of what the reference computes on this
path, used as the checker of the HIP kernels and nothing else. Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import it; the product package (``liteinfer_amd``) never does, and has
no CPU fallback that could route through it.

Modules:
  addressing  slot tables, newest slots, packed addresses and the KV
              slot-write (liteinfer/cache/block_pool.py:103-223,
              liteinfer/cache/kv_cache.py:236-253).
  attention   scaled dot-product attention over a paged pool, decode and
              packed/causal (liteinfer/models/attention.py:69-164), in any
              numpy float dtype (float64 is the reference answer).
  baseline    the dense eager / sdpa attention in torch fp32 on CPU threads,
              timed by bench.py as the CPU baseline.
  rope        rotary embedding with the reference's per-op roundings and the
              fused RoPE + slot-write (liteinfer/models/llama.py:79-98,
              :155-160).

How each function is pinned (tests/test_oracle.py):
  addressing.*        the reference's own known-answer vectors
                      (tests/unit/test_slot_table.py:30-155), committed as
                      tests/golden/addressing_kats.json, plus the closed form
                      slot = table[p // bs] * bs + p % bs on random tables.
  addressing.scatter  torch index_put_ on the same inputs (bit-exact) and the
                      invariant "untouched slots unchanged".
  attention.attend    a pure-Python scalar brute force (tests/golden/
                      make_golden.py, committed fixtures), torch's
                      scaled_dot_product_attention with is_causal on whole
                      prompts, and closed forms: one visible key gives its V
                      row; scale 0 gives the mean of the visible V rows; a
                      KV head whose V rows are all c gives c to exactly the
                      query heads h with h // groups == that head; chunk rows
                      equal the same rows of the whole prompt.
  baseline.*          agrees with attention.attend to fp32 rounding.
  rope.round_to       numpy's float16 conversion and, for bf16, torch's
                      float32 -> bfloat16 conversion on every float32 bit
                      pattern class (ties, carries into the exponent).
  rope.rope           torch's CPU ops x * cos + rotate_half(x) * sin in the
                      same dtype, bit for bit; exact cases: zero angle gives
                      x, a quarter turn gives rotate_half(x); in float64 each
                      (x[i], x[i + D/2]) pair keeps its length and two
                      rotations compose into the rotation by the sum of
                      their angles.
"""
