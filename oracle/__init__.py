"""CPU oracle for the AdaSplash / Lazy-Attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or as
the timed CPU baseline), never as the thing being measured on the GPU.

Everything here is plain numpy in float64 and restates the reference's
algorithms:

* ``entmax``    -- row-wise alpha-entmax: the bisection algorithm of the
  ``entmax`` package (called as ``entmax_bisect`` at
  tests/test_adasplash.py:53, tests/test_triton_entmax.py:24), exact
  sort-based closed forms for alpha=1.5 and alpha=2, and the Jacobian-vector
  product used by the backward.
* ``adasplash`` -- ``reference_attention`` of tests/test_adasplash.py:22-60
  plus its backward, the support set and the per-(128x64)-tile block mask.
* ``lazy``      -- the Lazy-Attention maths of lazy_attention_triton.py
  (forward :9-174, backward :180-497) in closed form.

Parity status of each function is stated in its docstring ("pinned by ...").
"""
