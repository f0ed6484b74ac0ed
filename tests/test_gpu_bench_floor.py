"""GPU: llmhip_bench_floor, the benchmark helper that streams rows in with
the register path's grid and access shape and does nothing else. Its
arguments are checked before anything is enqueued, and a launch over finite
logits writes nothing to `out`."""
import numpy as np
import pytest

from scriptonait_amd import sampler as smp

pytestmark = pytest.mark.gpu


def test_floor_launches_leave_out_untouched(sampler):
    import torch

    dev = torch.device("cuda:0")
    for V in (32000, 8192, 1000):
        lg = torch.randn((7, V), dtype=torch.float32, device=dev)
        out = torch.full((7,), 3.5, dtype=torch.float32, device=dev)
        sampler.bench_floor(lg, True, out)
        sampler.bench_floor(lg, False, out)
        torch.cuda.synchronize()
        assert (out.cpu().numpy() == 3.5).all()


@pytest.mark.parametrize("shape,V,why", [((4, 32772), None, "above the register path"),
                                         ((4, 1002), None, "not a multiple of 4"),
                                         ((4, 1000), 1004, "ld below V")])
def test_floor_refuses_shapes_the_kernel_does_not_take(sampler, shape, V, why):
    import torch

    lg = torch.zeros(shape, dtype=torch.float32, device="cuda:0")
    out = torch.zeros(shape[0], dtype=torch.float32, device="cuda:0")
    with pytest.raises(smp.SamplerError) as ei:
        sampler.bench_floor(lg, True, out, V=V)
    assert ei.value.status == -1, why
