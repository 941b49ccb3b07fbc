"""pi05_adarms_table_noalloc (include/pi05_denoise.h): the modulation table built without any
device allocation by the library, against the table pi05_refresh_weights builds in a context (the
same kernels: bit-exact) and against the oracle (fp32, 1e-5), on two calls in a row, the second
with a smaller input (fewer layers and steps), so the shared scratch is reused."""

from dataclasses import replace

import pytest
import torch

from oracle import denoise_oracle as O
from pi05_infer import _ext
from pi05_infer import synthetic as S
from pi05_infer.engine import OpenPi0InferConfig, OpenPi0Inference

pytestmark = pytest.mark.gpu


def _noalloc_table(w, g, steps):
    names = O.norm_dense_names(O.geometry_from(g))
    dev = torch.device("cuda")
    f = lambda n: w[n].float().to(dev).contiguous()  # noqa: E731
    dims = _ext.make_dims(g, 1, 16, steps)
    out = torch.full((steps, 2 * g.depth + 1, 3 * g.width), float("nan"), device=dev)
    _ext.adarms_table_noalloc(dims, f("time_mlp_in.weight"), f("time_mlp_in.bias"), f("time_mlp_out.weight"),
                              f("time_mlp_out.bias"), [f(a) for a, _ in names], [f(b) for _, b in names], out)
    return out


def _context_table(w, g, steps):
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=steps), g)
    model.load_state_dict(w)
    model.to("cuda")
    tab = model._context(1, 16, steps).adarms_table()
    torch.cuda.synchronize()
    model.close()
    return tab


@pytest.fixture(scope="module")
def weights():
    return S.make_weights(replace(S.ExpertGeometry(), depth=6))


def test_noalloc_table_matches_context_twice(weights):
    for depth, steps in ((6, 10), (2, 4)):
        print(f"no-alloc table: depth {depth}, {steps} steps", flush=True)
        g = replace(S.ExpertGeometry(), depth=depth)
        w = {k: v for k, v in weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < depth}
        got = _noalloc_table(w, g, steps)
        torch.cuda.synchronize()
        ref_ctx = _context_table(w, g, steps)
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref_ctx), f"depth {depth}, {steps} steps: differs from the context's table"
        ref = O.adarms_table(w, O.geometry_from(g), steps)
        torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-5)


def test_noalloc_rejects_more_steps_than_its_scratch():
    g = replace(S.ExpertGeometry(), depth=1)
    dims = _ext.make_dims(g, 1, 16, 33)
    z = torch.zeros(1, device="cuda")
    with pytest.raises(_ext.Pi05Error, match="PI05_E_INVALID.*no-alloc scratch maximum of 32 steps"):
        _ext.adarms_table_noalloc(dims, z, z, z, z, [z] * 3, [z] * 3, torch.zeros(33, 3, 3072, device="cuda"))
