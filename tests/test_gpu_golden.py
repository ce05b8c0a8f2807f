"""The HIP path against the committed small fixture (routing bit-exact, layer
outputs and gradients within the bf16 bar)."""

import os

import numpy as np
import pytest
import torch

from placemoe_amd import experts, kernels
from tests.helpers import assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_gpu_matches_golden_fixture(cuda):
    v = dict(np.load(os.path.join(GOLDEN, "oracle_small.npz")))
    bf = lambda a, grad=False: torch.as_tensor(a).to(torch.bfloat16).to(cuda).requires_grad_(grad)  # noqa: E731
    C = v["slot_to_logical"].size
    M = torch.as_tensor(v["mapping"]).to(cuda)
    src = torch.as_tensor(v["sources"]).to(cuda)
    sel = torch.as_tensor(v["selected"]).to(cuda)
    r = kernels.route(sel, C, mapping=M, sources=src)
    for name in ("phys", "counts", "offsets", "pos"):
        assert_exact(getattr(r, name), v[name], name)
    x, w, fc1, fc2 = bf(v["hidden"], True), bf(v["routing_weights"], True), bf(v["fc1"], True), bf(v["fc2"], True)
    out = experts.expert_layer(x, w, sel, fc2, fc1_1_2_weight=fc1, mapping=M, sources=src)
    out.backward(bf(v["grad_out"]))
    ref = lambda n: torch.as_tensor(v[n])  # noqa: E731
    assert_bf16_close(out, ref("out"), name="out")
    assert_bf16_close(x.grad, ref("dx"), name="dx")
    assert_bf16_close(w.grad, ref("dw"), name="dw")
    assert_bf16_close(fc1.grad, ref("dw1"), name="dw1")
    assert_bf16_close(fc2.grad, ref("dw2"), name="dw2")
