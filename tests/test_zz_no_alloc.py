"""rxmet_qdq_backward_noalloc (no workspace, no device allocation: the encoding-gradient
partials live in a file-scope device array) against rxmet_qdq_backward with a workspace:
dx and both encoding gradients bit for bit, on two calls in a row of which the second is
smaller, for the run layout (per-tensor, per-channel rows) and the column layout."""
import numpy as np
import pytest
import torch

import rxmet_lib

pytestmark = pytest.mark.gpu

# (outer, C, inner) pairs: a call, then a smaller one on the same scratch
CASES = [
    ((1, 1, 8192 * 1024), (1, 1, 300001)),      # per-tensor, long runs
    ((1, 512, 4096), (1, 64, 1000)),            # per-channel over dim 0
    ((2048, 16, 8), (100, 16, 3)),              # encodings on an inner axis: column layout
]


def _run(cuda, layout, seed, mode, noalloc):
    outer, C, inner = layout
    n = outer * C * inner
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, generator=g) * 2).to(cuda)
    gr = torch.randn(n, generator=g).to(cuda)
    s = (torch.rand(C, generator=g) * 0.05 + 0.01).to(cuda)
    o = torch.round(torch.rand(C, generator=g) * 20 - 10).to(cuda)
    dx = torch.empty_like(x)
    enc = mode == 0
    ds = torch.full((C,), 7.0, device=cuda) if enc else None
    do = torch.full((C,), 7.0, device=cuda) if enc else None
    stream = torch.cuda.current_stream().cuda_stream
    ptr = lambda t: None if t is None else t.data_ptr()
    if noalloc:
        rxmet_lib.call("rxmet_qdq_backward_noalloc", x.data_ptr(), gr.data_ptr(), dx.data_ptr(),
                       ptr(ds), ptr(do), outer, C, inner, s.data_ptr(), o.data_ptr(), -128, 127,
                       mode, stream)
    else:
        nb = rxmet_lib.load().rxmet_qdq_workspace_bytes(outer, C, inner)
        ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=cuda)
        rxmet_lib.call("rxmet_qdq_backward", x.data_ptr(), gr.data_ptr(), dx.data_ptr(), ptr(ds),
                       ptr(do), outer, C, inner, s.data_ptr(), o.data_ptr(), -128, 127, mode,
                       ws.data_ptr(), stream)
    torch.cuda.synchronize()
    return [t.cpu() for t in (dx, ds, do) if t is not None]


@pytest.mark.parametrize("pair", CASES)
@pytest.mark.parametrize("mode", [0, 1])
def test_noalloc_backward_equals_workspace_backward(cuda, pair, mode):
    print(f"[qdq noalloc] layouts={pair} mode={mode}", flush=True)
    for k, layout in enumerate(pair):
        ref = _run(cuda, layout, 40 + k, mode, noalloc=False)
        got = _run(cuda, layout, 40 + k, mode, noalloc=True)
        for a, b in zip(got, ref):
            assert torch.equal(a, b), (layout, mode)
        if mode == 0:
            assert torch.isfinite(got[1]).all() and (got[1] != 7.0).all()
