"""The HIP path against the committed small fixtures (routing bit-exact, layer
outputs and gradients within the bf16 bar, or the fp16 bar for the fp16
fixture)."""

import os

import numpy as np
import pytest
import torch

from placemoe_amd import experts, kernels
from tests.helpers import BF16_REL, FP16_REL, assert_bf16_close, assert_exact

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name,dtype,rel", [("oracle_small.npz", torch.bfloat16, BF16_REL),
                                            ("oracle_small_f16.npz", torch.float16, 1.5 * FP16_REL)])
def test_gpu_matches_golden_fixture(cuda, name, dtype, rel):
    v = dict(np.load(os.path.join(GOLDEN, name)))
    bf = lambda a, grad=False: torch.as_tensor(a).to(dtype).to(cuda).requires_grad_(grad)  # noqa: E731
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
    assert out.dtype == dtype
    assert_bf16_close(out, ref("out"), rel=rel, name="out")
    assert_bf16_close(x.grad, ref("dx"), rel=rel, name="dx")
    assert_bf16_close(w.grad, ref("dw"), rel=rel, name="dw")
    assert_bf16_close(fc1.grad, ref("dw1"), rel=rel, name="dw1")
    assert_bf16_close(fc2.grad, ref("dw2"), rel=rel, name="dw2")
