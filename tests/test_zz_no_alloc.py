"""cvmm_sort_routes_noalloc (the sort with a static device scratch, for
callers that cannot allocate) gives the bits of cvmm_sort_routes, call after
call on one GPU: the scratch keeps the previous call's contents, so a second,
smaller call must not see them."""
from __future__ import annotations

import pytest
import torch

from cvmm_codex_amd import _native as N

pytestmark = pytest.mark.gpu


def _outputs(R, E):
    f = lambda n, dt: torch.full((n,), -7, dtype=dt, device="cuda")
    return dict(ssel=f(R, torch.int32), perm=f(R, torch.int64), tok=f(R, torch.int64), off=f(E, torch.int64),
                pos=f(R, torch.int32), nin=f(1, torch.int32))


def _sort(lib, raw, is64, R, E, k, o, ws=None):
    st = N.stream_of(raw.device)
    outs = (N.ptr(o["ssel"]), N.ptr(o["perm"]), N.ptr(o["tok"]), N.ptr(o["off"]), N.ptr(o["pos"]), N.ptr(o["nin"]))
    if ws is None:
        return lib.cvmm_sort_routes_noalloc(N.ptr(raw), is64, R, E, k, *outs, st)
    return lib.cvmm_sort_routes(N.ptr(raw), is64, R, E, k, *outs, N.ptr(ws), ws.numel(), st)


@pytest.mark.parametrize("sizes", [
    [(65536, 64, 8, 1), (4000, 16, 4, 1)],                  # ff_up size, then a smaller one
    [(524288, 256, 64, 1), (1000, 7, 1, 0)],               # SwitchHead size (column scan), then int32 ids
    [(70000, 32767, 2, 1), (3000, 8192, 2, 1), (5, 3, 1, 0)],   # the largest expert count, then smaller
])
def test_noalloc_sort_matches_the_workspace_sort(sizes):
    lib = N.lib()
    for i, (R, E, k, is64) in enumerate(sizes):
        g = torch.Generator().manual_seed(1000 * i + R + E)
        raw = torch.randint(-1, E + 1, (R,), generator=g, dtype=torch.int64 if is64 else torch.int32).cuda()
        a, b = _outputs(R, E), _outputs(R, E)
        ws = torch.empty(lib.cvmm_sort_workspace_bytes(R, E), dtype=torch.uint8, device="cuda")
        N.check(_sort(lib, raw, is64, R, E, k, a, ws), "cvmm_sort_routes")
        N.check(_sort(lib, raw, is64, R, E, k, b), "cvmm_sort_routes_noalloc")
        torch.cuda.synchronize()
        for n in a:
            assert torch.equal(a[n], b[n]), (i, R, E, n)
        assert int((b["off"][-1]).item()) + int(b["nin"].item()) == R


def test_noalloc_sort_twice_in_a_row_on_the_same_outputs():
    """Two calls back to back, the second smaller, without a sync between."""
    lib = N.lib()
    g = torch.Generator().manual_seed(5)
    big = torch.randint(0, 64, (65536,), generator=g).cuda()
    small = torch.randint(0, 10, (777,), generator=g).cuda()
    o1, o2 = _outputs(65536, 64), _outputs(777, 10)
    N.check(_sort(lib, big, 1, 65536, 64, 8, o1), "first")
    N.check(_sort(lib, small, 1, 777, 10, 3, o2), "second")
    r1, r2 = _outputs(65536, 64), _outputs(777, 10)
    for raw, R, E, k, r in ((big, 65536, 64, 8, r1), (small, 777, 10, 3, r2)):
        ws = torch.empty(lib.cvmm_sort_workspace_bytes(R, E), dtype=torch.uint8, device="cuda")
        N.check(_sort(lib, raw, 1, R, E, k, r, ws), "reference")
    torch.cuda.synchronize()
    for n in o1:
        assert torch.equal(o1[n], r1[n]), n
        assert torch.equal(o2[n], r2[n]), n
