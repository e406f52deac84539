"""mi_attn_bwd_noalloc (workspace in the library's static device array) against
mi_attn_bwd (caller's workspace): the same kernels, so dQ, dK and dV must
be bit-identical.  Two calls in a row, the second with a smaller input (the
array keeps the first call's workspace); D = 16, 32, 64 and 128, causal and not,
sequence lengths with and without a partial last tile; the
size limit is refused before anything is enqueued."""
import math

import pytest
import torch

from gpu_ref import seeded

pytestmark = pytest.mark.gpu


def _inputs(gpu, B, H, S, D, seed):
    from gpt_from_scratch_amd import flash_attn_forward
    q, k, v, do = (seeded((B, H, S, D), seed + i).to(gpu) for i in range(4))
    o, lse = flash_attn_forward(q, k, v, True)
    return q, k, v, o, do, lse


def test_noalloc_backward_matches_workspace_backward(gpu):
    from gpt_from_scratch_amd import _lib
    for B, H, S, D, causal in ((2, 6, 1024, 64, True), (1, 3, 256, 128, False),
                               (1, 2, 192, 64, True), (1, 4, 320, 32, True),
                               (2, 2, 128, 16, False), (1, 3, 100, 64, True),
                               (1, 2, 77, 128, False)):
        q, k, v, o, do, lse = _inputs(gpu, B, H, S, D, 300 + S + D)
        scale = 1.0 / math.sqrt(D)
        want = [torch.empty_like(q) for _ in range(3)]
        ws = _lib.bwd_workspace(lse)
        _lib.attn_bwd(q, k, v, o, do, lse, ws, *want, causal, scale)
        got = [torch.full_like(q, float("nan")) for _ in range(3)]
        _lib.attn_bwd_noalloc(q, k, v, o, do, lse, *got, causal, scale)
        torch.cuda.synchronize()
        for name, g, w in zip(("dq", "dk", "dv"), got, want):
            assert torch.equal(g, w), (name, B, H, S, D, causal)


def test_noalloc_refuses_more_rows_than_its_array(gpu):
    """Sizes beyond the static workspace are refused from the sizes alone (the
    tensor pointers are NULL, which the full validation would refuse too)."""
    from gpt_from_scratch_amd import _lib
    lib = _lib.lib()
    st4 = (torch.zeros(4, dtype=torch.int64) + 1).tolist()
    arr = lambda: _lib._i64x4()(*st4)
    S = _lib.NOALLOC_MAX_ROWS + 64
    stream = _lib._stream(torch.empty(1, device=gpu))
    st = lib.mi_attn_bwd_noalloc(2, 1, 1, S, 64, 1, 0.125,
                                 None, arr(), None, arr(), None, arr(), None, arr(), None, arr(),
                                 None, None, arr(), None, arr(), None, arr(), stream)
    assert st == 1 and b"MI_ATTN_NOALLOC_MAX_ROWS" in lib.mi_last_error()


def test_noalloc_backward_replays_under_graph_capture(gpu):
    """After one call outside capture (the per-device address lookup), the call
    is captured into a graph; every replay, with eager work between replays,
    reproduces mi_attn_bwd bit for bit."""
    from gpt_from_scratch_amd import _lib
    B, H, S, D = 2, 4, 512, 64
    q, k, v, o, do, lse = _inputs(gpu, B, H, S, D, 900)
    scale = 1.0 / math.sqrt(D)
    want = [torch.empty_like(q) for _ in range(3)]
    _lib.attn_bwd(q, k, v, o, do, lse, _lib.bwd_workspace(lse), *want, True, scale)
    got = [torch.empty_like(q) for _ in range(3)]
    _lib.attn_bwd_noalloc(q, k, v, o, do, lse, *got, True, scale)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.attn_bwd_noalloc(q, k, v, o, do, lse, *got, True, scale)
    for replay in range(3):
        for t in got:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, g, w in zip(("dq", "dk", "dv"), got, want):
            assert torch.equal(g, w), (name, replay)
