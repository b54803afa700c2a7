"""Linear's cast cache under bf16/f16 autocast (4d_ttt_merging_amd/layers.py).

Without autograd, `Linear` and `LinearKMaskedBias` keep one autocast-dtype copy
of their weight and bias.  The products must equal autocast's own F.linear bit
for bit, and every change of the parameters (in place, by load_state_dict, by
`.data` writes followed by `clear_cast_cache`) must be seen.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.conftest import import_package

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layers():
    return import_package("layers")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("masked", [False, True])
def test_linear_cast_cache_equals_autocast(layers, device, dtype, masked):
    print(f"[linear cache] dtype={dtype} masked={masked}", flush=True)
    torch.manual_seed(0)
    cls = layers.LinearKMaskedBias if masked else layers.Linear
    lin = cls(256, 768, bias=True, device=device)
    torch.nn.init.normal_(lin.bias)

    def autocast_linear(x):
        bias = lin.bias * lin.bias_mask if masked else lin.bias
        with torch.autocast("cuda", dtype=dtype):
            return F.linear(x, lin.weight, bias)

    def cached(x):
        with torch.autocast("cuda", dtype=dtype):
            return lin(x)

    x = torch.randn(300, 256, device=device)
    with torch.no_grad():
        first = cached(x)
        assert "_cast_cache" in lin.__dict__
        assert first.dtype == dtype
        assert torch.equal(first, autocast_linear(x))
        assert torch.equal(cached(x), first)

        lin.weight.mul_(0.5)  # in place: the version counter moves
        halved = cached(x)
        assert torch.equal(halved, autocast_linear(x)) and not torch.equal(halved, first)

        state = {k: v.clone() for k, v in lin.state_dict().items()}
        state["bias"].add_(1.0)
        lin.load_state_dict(state)
        assert torch.equal(cached(x), autocast_linear(x))

        lin.weight.data.mul_(2.0)  # bypasses the version counter
        lin.clear_cast_cache()
        assert torch.equal(cached(x), autocast_linear(x))

        # fp32 (no autocast) runs the parameters as they are
        assert torch.equal(lin(x), F.linear(x, lin.weight, lin.bias * lin.bias_mask if masked else lin.bias))

    # copies made under inference_mode serve no_grad calls, and the other way round
    lin.clear_cast_cache()
    with torch.inference_mode(), torch.autocast("cuda", dtype=dtype):
        inf = lin(x)
    with torch.no_grad(), torch.autocast("cuda", dtype=dtype):
        assert torch.equal(lin(x), inf)
    lin.clear_cast_cache()
    with torch.no_grad(), torch.autocast("cuda", dtype=dtype):
        ng = lin(x)
    with torch.inference_mode(), torch.autocast("cuda", dtype=dtype):
        assert torch.equal(lin(x), ng)

    lin.clear_cast_cache()
    with torch.autocast("cuda", dtype=dtype):
        out = lin(x)  # autograd on: no cached copies
    assert "_cast_cache" not in lin.__dict__ and out.requires_grad


@pytest.mark.parametrize("masked", [False, True])
def test_linear_cast_cache_off_under_capture_and_cache_disabled(layers, device, masked):
    """A graph captured with no warm-up casts inside the graph (no cached copy is built
    during capture), an eager call before any replay equals plain autocast, every replay
    sees an in-place parameter update made after the capture, and with autocast's cast
    cache switched off no copy is kept."""
    print(f"[linear cache] graph capture, masked={masked}", flush=True)
    torch.manual_seed(1)
    cls = layers.LinearKMaskedBias if masked else layers.Linear
    lin = cls(256, 768, bias=True, device=device)
    torch.nn.init.normal_(lin.bias)
    x = torch.randn(200, 256, device=device)

    def plain():
        bias = lin.bias * lin.bias_mask if masked else lin.bias
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return F.linear(x, lin.weight, bias)

    def call():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return lin(x)

    # The GEMM library's handle and workspace come from a plain product on a side
    # stream (torch's capture pattern); the module itself is not called before capture.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        plain()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = call()
    assert "_cast_cache" not in lin.__dict__
    eager = call()  # before any replay
    assert torch.equal(eager, plain())
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(static, plain())
    with torch.no_grad():
        lin.weight.mul_(0.25)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(static, plain()) and not torch.equal(static, eager)
    assert torch.equal(call(), plain())

    lin.clear_cast_cache()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
        out = lin(x)
    assert "_cast_cache" not in lin.__dict__
    assert torch.equal(out, plain())
