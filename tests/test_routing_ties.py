"""Probability ties built on the host (the router the GPU test
test_gpu_routing_exact.py::test_probability_ties_decided_as_the_reference_does
runs through every device path).

The reference ranks experts by p = fl(e / S), e = std::exp(fl(L - m)), S
the fp32 sum of every e in id order, the lower id first among equal p
(src/cpu/reference_ops.cpp:135-196). The construction must produce, for
each kind of tie, exactly the outcome that rule gives, checked here on the
oracle and on the reference's own compiled CPU code (oracle/_ref)."""

import numpy as np

import oracle as O
from test_gpu_routing_exact import D, E, K, tie_router


def test_tie_router_construction():
    # The oracle's logits are the targets, and its ids show the reference's
    # tie rule on every pair: the lower logit first where p ties, the higher
    # one where the exps are one ulp apart and p does not tie, and at the
    # k-th pick the lower logit picked and the higher one left out.
    bits, router_f, x, pairs, logits = tie_router(np.random.default_rng(11))
    ora = O.route_qwen_top_k(x, router_f, D, E, K, True)
    assert np.array_equal(ora["logits"], logits)
    pos = {int(e): i for i, e in enumerate(ora["ids"])}
    for name in ("exp_tie", "key_tie", "quot_tie"):
        lo, hi = pairs[name]
        assert logits[lo] < logits[hi] and pos[lo] + 1 == pos[hi], (name, pos.get(lo), pos.get(hi))
    lo, hi = pairs["quot_nontie"]
    assert pos[hi] + 1 == pos[lo]
    lo, hi = pairs["boundary_tie"]
    assert pos[lo] == K - 1 and hi not in pos
    if O.ref_available():
        assert np.array_equal(O.route_qwen_top_k(x, router_f, D, E, K, True, impl="ref")["ids"], ora["ids"])
