"""The no-allocation decode entry (oscar_paged_decode_noalloc) against the
workspace entry (oscar_paged_decode), through the C ABI.

Both run the same kernels on the same inputs (the split partials live in the
library's device scratch instead of a caller workspace), so the outputs must
be bit-identical.  Two calls in a row, the second with a smaller input (the
scratch keeps the first call's partials), and a launch whose partials would
exceed the 32 MiB scratch is rejected before anything is enqueued.
"""
import pytest
import torch

from oscar_amd.kernels import _lib, decode
from tests.scenarios import decode_case

pytestmark = pytest.mark.gpu

WORKSPACE_TOO_SMALL = -3


def noalloc_entry():
    return _lib.load().oscar_paged_decode_noalloc


def both_entries(case, device):
    L = case.layer
    q, k, v = case.rotated()
    stage = tuple(t.to(device) for t in L.stage())
    p = decode.plan(q.to(device), k.to(device), v.to(device), L.k_cache.to(device), L.v_cache.to(device),
                    case.bt.to(device), case.qsl, case.seqs, L.scale, stage)
    want = p.launch().clone()
    common = p.args[:-3]                           # everything before (out, workspace, workspace_size)
    got = torch.full_like(want, float("nan"))
    status = noalloc_entry()(*common, got.data_ptr(), _lib.stream_handle(got.device))
    torch.cuda.synchronize()
    assert status == 0
    return got, want, p


def test_noalloc_matches_workspace_entry_twice(device):
    got, want, _ = both_entries(decode_case([24579], [4], seed=93), device)
    assert torch.equal(got, want)
    # second call, smaller: 2 requests, 32-token pages
    got, want, p = both_entries(decode_case([300, 5], [2, 1], bs=32, seed=2, sink=32, recent=32, staging=64), device)
    assert torch.equal(got, want)
    # partials beyond the scratch: rejected, nothing enqueued
    args = list(p.args[:-3])
    args[23], args[24] = 16, 1 << 19             # max_query_len, max_history: 51 MB of partials
    out = torch.full_like(want, 7.0)
    status = noalloc_entry()(*args, out.data_ptr(), _lib.stream_handle(out.device))
    torch.cuda.synchronize()
    assert status == WORKSPACE_TOO_SMALL
    assert (out == 7.0).all()
