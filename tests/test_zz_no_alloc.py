"""macai_gdr_forward_noalloc, through the C ABI: the inference forward with its per-chunk operands in the library's
fixed device array instead of a caller's workspace.  Two calls in a row, the second smaller, each give the bits of
macai_gdr_forward with a freshly allocated workspace; a shape over the array's size is refused before any launch."""
import pytest
import torch

from macai.gated_delta import _native as N
from oracle import gdr

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, Hk, DK, DV, dtype, seed):
    inp = gdr.make_inputs(B, T, Hk, H, DK, DV, dtype, s0=True, seed=seed)
    q, k = (inp[n][:, :, ::H // Hk].contiguous().cuda() for n in ("query", "key"))
    return [q, k] + [inp[n].cuda() for n in ("value", "g", "beta", "initial_state")]


def _forward(noalloc, xs, B, T, H, Hk, DK, DV, dtype):
    q, k, v, g, beta, s0 = xs
    P, code, st = N.ptr, N.dtype_code(dtype), N.stream_of(q)
    o = torch.full((B, T, H, DV), float("nan"), dtype=dtype, device="cuda")
    sT = torch.full((B, H, DK, DV), float("nan"), device="cuda")
    head = (P(q), P(k), P(v), P(g), P(beta), P(s0), P(o), P(sT))
    tail = (B, T, H, Hk, DK, DV, code, 1, DK ** -0.5, 0, None, 0, st)
    if noalloc:
        N.call("macai_gdr_forward_noalloc", *head, *tail)
    else:
        nbytes = N.lib().macai_gdr_forward_workspace(B, T, H, DK, DV, code, 0)
        ws = torch.full((nbytes,), 255, dtype=torch.uint8, device="cuda")
        N.call("macai_gdr_forward", *head, P(ws), nbytes, *tail)
    torch.cuda.synchronize()
    return o, sT


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_forward_matches_the_workspace_forward(dtype):
    big, small = (4, 1024, 16, 16, 128, 128), (2, 130, 4, 2, 128, 128)
    if dtype == torch.float32:
        big = (2, 1024, 16, 16, 128, 128)        # float32 operands take twice the bytes: half the rows still fit
    for i, shape in enumerate((big, small)):
        print("case noalloc forward", shape, dtype, flush=True)
        B, T, H, Hk, DK, DV = shape
        need = N.lib().macai_gdr_forward_workspace(B, T, H, DK, DV, N.dtype_code(dtype), 0)
        assert need <= N.NOALLOC_SCRATCH_BYTES
        xs = _inputs(*shape, dtype, seed=40 + i)
        o1, s1 = _forward(True, xs, *shape, dtype)
        o2, s2 = _forward(False, xs, *shape, dtype)
        assert not torch.isnan(o1).any() and not torch.isnan(s1).any()
        assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_noalloc_forward_refuses_shapes_over_its_scratch():
    B, T, H, DK, DV = 8, 4096, 32, 128, 128
    need = N.lib().macai_gdr_forward_workspace(B, T, H, DK, DV, N.BF16, 0)
    assert need > N.NOALLOC_SCRATCH_BYTES
    p = 1 << 20
    with pytest.raises(ValueError, match="fixed"):
        N.call("macai_gdr_forward_noalloc", *([p] * 6), p, p, B, T, H, H, DK, DV, N.BF16, 1, 1.0, 0, None, 0, None)


def test_noalloc_forward_under_graph_capture():
    """The entry point for code under HIP graph capture: after one call on the device (which looks up the array's
    address), the call is captured into a graph (torch.cuda.CUDAGraph) and replayed three times, with eager work on
    the same buffers between the replays; every replay gives the bits of macai_gdr_forward with a workspace."""
    shape, dtype = (2, 300, 4, 2, 128, 128), torch.bfloat16
    print("case noalloc forward captured", shape, dtype, flush=True)
    B, T, H, Hk, DK, DV = shape
    xs = _inputs(*shape, dtype, seed=47)
    ref_o, ref_s = _forward(False, xs, *shape, dtype)
    q, k, v, g, beta, s0 = xs
    o = torch.empty(B, T, H, DV, dtype=dtype, device="cuda")
    sT = torch.empty(B, H, DK, DV, device="cuda")
    P, code = N.ptr, N.dtype_code(dtype)
    args = (P(q), P(k), P(v), P(g), P(beta), P(s0), P(o), P(sT), B, T, H, Hk, DK, DV, code, 1, DK ** -0.5, 0, None, 0)
    N.call("macai_gdr_forward_noalloc", *args, N.stream_of(q))   # the first call on the device, outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        N.call("macai_gdr_forward_noalloc", *args, N.stream_of(q))
    for _ in range(3):
        o.fill_(float("nan"))
        sT.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, ref_o) and torch.equal(sT, ref_s)
