"""CPU oracle for the Strata hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with torch, what the reference computes on
the path the HIP library replaces: NATTEN 0.21.5 ``na3d`` (clamped windows,
dilation), the stereographic RoPE of physicsnemo's Strata attention, and the
pre-norm Strata block.  Neither NATTEN nor physicsnemo is installable here, so
the restatement follows their published semantics and the reference's call
sites (cited per function).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
reported CPU baseline.  The product (``strata_amd``) never imports it.

Pinning (what makes each function trustworthy beyond re-typing a formula):
  * ``na3d``: equals ``na3d_bruteforce`` (window = the feasible length-k run
    nearest the query, found by search) and ``na3d_unfold`` (torch unfold of
    the keys); equals dense SDPA when the kernel covers the grid; kernel 1
    returns v; committed golden vectors from the brute-force form.
  * ``rope``: closed forms of the stereographic projection (equator, pole,
    centre), rotation norm preservation, relative-position property.
  * ``block``: composition of the pinned parts with torch's own Linear,
    LayerNorm and GELU; zero-weight identities.
"""
