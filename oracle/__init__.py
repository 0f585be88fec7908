"""CPU oracle for the MoE expert path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's MoE expert
path (``mxfp4_expert.py`` and ``streamed_moe_router.py``) so that the HIP
kernels can be checked against it on identical seeded inputs.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker: nothing in the product path
(``kcapw-klcquant_amd/``) imports or calls it, and there is no CPU fallback.

Modules and what pins them (tests/test_oracle_*.py):

* ``numerics``  — float32 -> bfloat16 / float16 rounding.  Pinned against
  hand-worked bit patterns (ties to even, overflow, subnormals, NaN) and
  against numpy's own float16 cast.
* ``mxfp4``     — MXFP4 -> dense dequant (mxfp4_expert.py:17-34, 357-379).
  Pinned against the E2M1/E8M0 definitions of the OCP MX v1.0 spec evaluated
  with ``math.ldexp`` for all 16 codes x 256 scale bytes, the reference's
  FP4_VALUES table, and single-nibble probes for the layout.
* ``router``    — router logits, top-k, softmax, dispatch
  (streamed_moe_router.py:268-284, 365-375).  Pinned by exact rational
  dot products (``fractions``), brute-force selection and closed-form
  softmax cases, and against torch's own CPU results on the golden vectors
  of tests/golden/ (ids, tie order, bf16 weights, combine bits).
* ``torch_cpu`` — the torch CPU kernels the router calls: top-k's libstdc++
  order of equal values and the float32 softmax with SLEEF's expf.  Pinned
  directly against ``torch.topk`` / ``torch.softmax`` (tie-heavy rows, the
  partial-sort regime, adversarial rows past the introselect depth limit).
* ``experts``   — gate_up / clamped SwiGLU / down / weighted combine
  (streamed_moe_router.py:483-529) and the bias-only fallback (:317-322).
  Pinned by clamp special cases, exact rational GEMVs on tiny shapes and
  order-sensitive bfloat16 combine cases.
* ``layer``     — one MoE layer for a batch of tokens, composing the above.
* ``rmsnorm``   — streamed_attention.py:27-28 (the stacked workload only).

Parity of every function above is pinned; no function is "parity unpinned".
Equal bfloat16 logits come out in torch.topk's CPU order (``torch_cpu``).  The
one documented divergence is the router's accumulation: the logits are the
correctly rounded bf16(f32(x . w) + b), where torch's F.linear accumulates in
float32 and lands one bf16 ulp away on a few tokens; the golden vectors record
every such logit, and tests/golden/router_boundary.npz the crafted routers on
which it changes the routing.
"""
