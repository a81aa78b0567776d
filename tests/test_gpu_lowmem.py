"""Low-memory grad-input (cvmm.py:1228-1338, :1605-1634): a token-input
unweighted top-k sum that goes through the [R, d_in] route buffer can run
over slices of its top-k columns (cvmm_lowmem_chunk_size), each sorted on
its own with a buffer of T * chunk rows, summed in fp32 and rounded once, so
the gradients keep the bits of the one-call sum; and when the one-call
workspace does not fit, the backward falls back to slices instead of
raising.  The dense top-k sum (no route buffer) is switched off here so the
route-buffer path is the one exercised."""
import pytest
import torch

import cvmm_codex_amd.api as C
from cvmm_codex_amd import _native as N

pytestmark = pytest.mark.gpu


def _case(T, E, k, d_in, d_out, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d_in, generator=g).to(torch.bfloat16)
    keys = torch.randn(E, d_in, d_out, generator=g) / d_in ** 0.5
    sel = torch.rand(T, E, generator=g).topk(k, dim=-1).indices
    sel[::7, 1] = E + 3          # some out-of-range ids: left out of every sum
    gy = torch.randn(T, k, d_out, generator=g).to(torch.bfloat16)
    return x.cuda(), keys.cuda(), sel.cuda(), gy.cuda()


def _backward(x, keys, sel, gy, chunk):
    old = C.cvmm_lowmem_chunk_size
    C.cvmm_lowmem_chunk_size = chunk
    try:
        xg = x.clone().requires_grad_(True)
        kg = keys.clone().requires_grad_(True)
        s = C.cvmm_prepare_sel2(sel)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = C.cvmm(xg, s, kg)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        y.backward(gy)
        torch.cuda.synchronize()
        return xg.grad, kg.grad, torch.cuda.max_memory_allocated() - base
    finally:
        C.cvmm_lowmem_chunk_size = old


@pytest.fixture
def route_buffer():
    lib = N.lib()
    assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 1) == 0
    yield
    lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)


@pytest.mark.parametrize("chunk", [16, 5, 1])
def test_lowmem_slices_keep_the_bits_with_less_memory(route_buffer, chunk):
    x, keys, sel, gy = _case(2048, 256, 64, 512, 64, 11)
    gx0, gk0, peak0 = _backward(x, keys, sel, gy, 0)
    gx1, gk1, peak1 = _backward(x, keys, sel, gy, chunk)
    assert torch.equal(gx0, gx1)
    assert torch.equal(gk0, gk1)
    # the one-call route buffer is 2048 * 64 rows of 512 bf16 values (134 MB)
    assert peak1 < peak0 - 64 * 2048 * 512 * 2 // 2, (peak0, peak1)


def test_oom_on_the_route_buffer_falls_back_to_slices(route_buffer):
    """SwitchHead V shapes (T = 8192, top-64 of 256, d_in = 2048): the
    one-call route buffer is 2.1 GB.  With the allocator capped ~1 GB above
    what the backward holds otherwise, that workspace raises
    OutOfMemoryError; the backward takes slices (32 columns still do not
    fit, 16 do) and gives the one-call bits."""
    x, keys, sel, gy = _case(8192, 256, 64, 2048, 64, 12)
    gx0, gk0, _ = _backward(x, keys, sel, gy, 0)
    gx1, gk1, _ = _backward(x, keys, sel, gy, 16)       # warms the kept workspaces
    assert torch.equal(gx0, gx1) and torch.equal(gk0, gk1)
    del gx1, gk1
    torch.cuda.empty_cache()
    total = torch.cuda.get_device_properties(0).total_memory
    cap = torch.cuda.memory_allocated() + (1 << 30)
    torch.cuda.set_per_process_memory_fraction(cap / total)
    try:
        with pytest.raises(torch.OutOfMemoryError):     # the one-call route buffer cannot be had
            torch.empty(8192 * 64 * 2048 * 2, dtype=torch.uint8, device="cuda")
        gx2, gk2, _ = _backward(x, keys, sel, gy, 0)
    finally:
        torch.cuda.set_per_process_memory_fraction(1.0)
    assert torch.equal(gx0, gx2)
    assert torch.equal(gk0, gk2)
