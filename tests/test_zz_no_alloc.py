"""The allocation-free attention entry point, vgo_mass_bias_attn_fwd_static.

It runs the kernels of vgo_mass_bias_attn_fwd_ws with the library's static
device scratch in place of a caller's workspace, so its output must equal the
workspace entry's bit for bit.  Two calls in a row (the second smaller) check
that the scratch's leftover contents from the first call do not leak into the
second.  The size limit is checked on the host before any launch.  A call
allocates nothing (torch's allocator and the device's free memory are unchanged
across it), and the entry captured into a HIP graph replays correctly with other
calls on the same scratch between the replays.
"""
from __future__ import annotations

import ctypes
import re

import pytest
import torch

from tests.conftest import ROOT, import_package

HEADER = ROOT / "include" / "vgo.h"


def _limit() -> int:
    m = re.search(r"#define VGO_ATTN_STATIC_SCRATCH_BYTES \((\d+)u \* 1024u \* 1024u\)", HEADER.read_text())
    return int(m.group(1)) << 20


def _args(lib_mod, q, k, v, bias, out):
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), None if bias is None else bias.data_ptr(),
            out.data_ptr(), q.shape[0], q.shape[1], q.shape[2], k.shape[2], 64,
            lib_mod.strides3(q), lib_mod.strides3(k), lib_mod.strides3(v), lib_mod.strides3(out),
            lib_mod.dtype_code(q.dtype))


def _run(entry: str, q, k, v, bias):
    lib_mod = import_package("_lib")
    lib = lib_mod.load()
    out = torch.full_like(q, float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    args = _args(lib_mod, q, k, v, bias, out)
    if entry == "static":
        lib_mod.check(lib.vgo_mass_bias_attn_fwd_static(*args, stream))
    else:
        need = ctypes.c_size_t(0)
        lib_mod.check(lib.vgo_mass_bias_attn_workspace(q.shape[0], q.shape[1], q.shape[2], k.shape[2],
                                                       lib_mod.dtype_code(q.dtype), ctypes.byref(need)))
        ws = torch.empty(max(need.value, 1) + 256, dtype=torch.uint8, device=q.device)
        base = ws.data_ptr() + (-ws.data_ptr()) % 256
        lib_mod.check(lib.vgo_mass_bias_attn_fwd_ws(*args, base, need.value, stream))
    return out


def _problem(seed, nq, nk, dtype, device, bias=True):
    g = torch.Generator(device=device).manual_seed(seed)
    q = (torch.randn(1, 16, nq, 64, device=device, generator=g) * 0.125).to(dtype)
    k = (torch.randn(1, 16, nk, 64, device=device, generator=g) * 0.125).to(dtype)
    v = torch.randn(1, 16, nk, 64, device=device, generator=g).to(dtype)
    b = None
    if bias:
        b = torch.randint(1, 9, (nk,), device=device, generator=g).float().log().to(dtype)
    return q, k, v, b


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_static_entry_equals_workspace_entry(device, dtype):
    # C4's merged attention (16,464 x 16,464), then a smaller ragged problem without bias
    # (fp32 runs the exact kernel, which needs no scratch; smaller shapes keep it quick)
    shapes = [(16464, 16464, True), (1000, 777, False)] if dtype != torch.float32 else \
        [(700, 900, True), (130, 257, False)]
    for i, (nq, nk, bias) in enumerate(shapes):
        print(f"[no-alloc] call {i}: {dtype} nq={nq} nk={nk} bias={bias}", flush=True)
        q, k, v, b = _problem(10 + i, nq, nk, dtype, device, bias)
        got = _run("static", q, k, v, b)
        ref = _run("ws", q, k, v, b)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), f"call {i}: static scratch result differs from the workspace entry"


@pytest.mark.gpu
def test_static_entry_rejects_problems_beyond_its_scratch(device):
    """A problem whose workspace exceeds the static scratch fails before any launch
    (NULL tensors: were the check missing, the null-pointer check would stop it)."""
    lib_mod = import_package("_lib")
    lib = lib_mod.load()
    need = ctypes.c_size_t(0)
    nk = 400_000  # V^T alone: 16 heads x 64 x 400,000 x 2 bytes = 819 MB
    lib_mod.check(lib.vgo_mass_bias_attn_workspace(1, 16, 512, nk, lib_mod.VGO_BF16, ctypes.byref(need)))
    assert need.value > _limit()
    s = lib_mod.strides3(torch.empty(1, 1, 1))
    status = lib.vgo_mass_bias_attn_fwd_static(None, None, None, None, None, 1, 16, 512, nk, 64, s, s, s, s,
                                               lib_mod.VGO_BF16, torch.cuda.current_stream().cuda_stream)
    assert status == lib_mod.VGO_EWORKSPACE
    assert "static" in lib_mod.last_error() and "vgo_mass_bias_attn_fwd_ws" in lib_mod.last_error()


@pytest.mark.gpu
def test_static_entry_allocates_nothing_and_replays_from_a_graph(device):
    """After its first call on a device, a call changes neither torch's allocated bytes
    nor the device's free memory (hipMemGetInfo); the entry captured into a HIP graph
    replays three times, with eager calls of another problem on the same scratch
    between the replays, and every replay equals the workspace entry bit for bit."""
    lib_mod = import_package("_lib")
    lib = lib_mod.load()
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    q, k, v, b = _problem(30, 3000, 2500, torch.bfloat16, device)
    ref = _run("ws", q, k, v, b)
    out = torch.full_like(q, float("nan"))
    args = _args(lib_mod, q, k, v, b, out)
    print("[no-alloc] eager call, then the allocation check", flush=True)
    lib_mod.check(lib.vgo_mass_bias_attn_fwd_static(*args, stream()))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    allocated, free = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
    lib_mod.check(lib.vgo_mass_bias_attn_fwd_static(*args, stream()))
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == allocated
    assert torch.cuda.mem_get_info()[0] == free
    assert torch.equal(out, ref)

    print("[no-alloc] capture into a HIP graph and replay", flush=True)
    captured = torch.full_like(q, float("nan"))
    cargs = _args(lib_mod, q, k, v, b, captured)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        lib_mod.check(lib.vgo_mass_bias_attn_fwd_static(*cargs, stream()))
    other = _problem(31, 700, 1900, torch.bfloat16, device, bias=False)
    other_ref = _run("ws", *other)
    for replay in range(3):
        captured.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, ref), f"replay {replay} differs from the workspace entry"
        assert torch.equal(_run("static", *other), other_ref)
        torch.cuda.synchronize()
