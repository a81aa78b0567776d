"""Host-side API semantics of cvmm_codex_amd.cvmm that need no GPU."""
import pytest
import torch

import cvmm_codex_amd as pkg
import cvmm_codex_amd.api as C


def _plain_sel():
    raw = torch.tensor([[2, 0], [1, 2]], dtype=torch.int32)
    ssel = torch.tensor([[0, 1], [2, 2]], dtype=torch.int32)
    perm = torch.tensor([1, 2, 0, 3])
    return C.CVMMSel(raw, ssel, perm // 2, perm)


def test_public_names():
    for name in ("CVMMSel", "cvmm_prepare_sel", "cvmm_prepare_sel2", "cvmm", "CVMM", "get_dtype",
                 "dtype_to_type_id", "create_kernels"):
        assert hasattr(pkg, name) and hasattr(C, name)
    for name in ("cvmm_expert_offsets_call", "cvmm_lowmem_chunk_size", "_cvmm_expert_offsets"):
        assert hasattr(C, name)


def test_cvmmsel_fields_and_clone():
    s = _plain_sel()
    c = s.clone()
    assert c is not s
    assert c.raw_sel is s.raw_sel and c.sel is s.sel and c.sel_index is s.sel_index
    assert c.out_index is s.out_index and c.reduction_weight is None
    s2 = C.CVMMSel(s.raw_sel, s.sel, s.sel_index)         # positional, defaults
    assert s2.out_index is None and s2.reduction_weight is None


def test_prepare_sel2_rewraps_cvmmsel():
    """cvmm.py:1788-1792: route input takes out_index (or sel_index)."""
    s = _plain_sel()
    w = torch.rand(2, 2)
    r = C.cvmm_prepare_sel2(s, w, route_input=True)
    assert r.sel_index is s.out_index and r.out_index is None and r.reduction_weight is w
    t = C.cvmm_prepare_sel2(s, w)
    assert t.sel_index is s.sel_index and t.out_index is s.out_index and t.reduction_weight is w
    rr = C.cvmm_prepare_sel2(r, None, route_input=True)  # route-major parent: sel_index
    assert rr.sel_index is r.sel_index


@pytest.mark.parametrize("route_input", [False, True])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_host_selectors_match_oracle(route_input, dtype):
    """cvmm_prepare_sel / cvmm_prepare_sel2 accept ids in host memory, as the
    reference's pure-torch versions do (cvmm.py:24-27, :1786-1803): the
    fields equal the oracle's (stable order among equal ids), with many ties."""
    import numpy as np
    from oracle import cvmm_oracle as O
    g = torch.Generator().manual_seed(5)
    sel = torch.randint(0, 7, (3, 11, 4), generator=g).to(dtype)
    w = torch.rand(3, 11, 4, generator=g)
    got = C.cvmm_prepare_sel2(sel, w, route_input=route_input)
    exp = O.prepare_sel2(sel.numpy(), w.numpy(), route_input=route_input)
    assert got.raw_sel.dtype == torch.int32 and got.sel.dtype == torch.int32
    np.testing.assert_array_equal(got.raw_sel.numpy(), exp.raw_sel)
    np.testing.assert_array_equal(got.sel.numpy(), exp.sel)
    np.testing.assert_array_equal(got.sel_index.numpy(), exp.sel_index)
    if route_input:
        assert got.out_index is None
    else:
        np.testing.assert_array_equal(got.out_index.numpy(), exp.out_index)
    assert got.reduction_weight is w
    one = C.cvmm_prepare_sel(sel, 7)
    e1 = O.prepare_sel(sel.numpy(), 7)
    np.testing.assert_array_equal(one.sel.numpy(), e1.sel)
    np.testing.assert_array_equal(one.sel_index.numpy(), e1.sel_index)
    assert one.out_index is None


def test_host_selector_is_a_snapshot():
    """Writing to the caller's ids after preparation changes nothing, as for a
    device selector."""
    sel = torch.tensor([[3, 1], [1, 0]], dtype=torch.int32)
    s = C.cvmm_prepare_sel2(sel)
    sel.fill_(9)
    assert s.raw_sel.tolist() == [[3, 1], [1, 0]]
    assert s.sel.tolist() == [[0, 1], [1, 3]]


def test_cpu_operands_are_rejected():
    """Only the selector metadata is made on the host: the product itself has
    no CPU path."""
    sel = C.cvmm_prepare_sel2(torch.zeros(3, 2, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        C.cvmm(torch.zeros(3, 4), sel, torch.zeros(2, 4, 5))


def test_dtype_ids_match_reference():
    assert C.dtype_to_type_id(torch.float32) == 0
    assert C.dtype_to_type_id(torch.float16) == 1
    assert C.dtype_to_type_id(torch.bfloat16) == 2
    with pytest.raises(ValueError):
        C.dtype_to_type_id(torch.int8)


def test_get_dtype_follows_autocast():
    assert C.get_dtype() == torch.float32


def test_storage_conversion_rules():
    f16 = torch.zeros(2, dtype=torch.float16)
    bf = torch.zeros(2, dtype=torch.bfloat16)
    assert C._storage_for(bf, torch.bfloat16) is bf
    assert C._storage_for(f16, torch.bfloat16).dtype == torch.float32
    assert C._storage_for(bf, torch.float32).dtype == torch.float32
    k = torch.zeros(3, 4, 5).transpose(1, 2)
    assert C._keys_view(k) is k                      # unit stride on d_in
    k2 = torch.zeros(3, 4, 5).permute(2, 0, 1).contiguous().permute(1, 2, 0)
    assert C._keys_view(k2) is k2
    k3 = torch.zeros(5, 4, 3).permute(2, 1, 0)[:, ::2, ::2]
    assert C._keys_view(k3).is_contiguous()


def test_cvmmsel_is_a_dataclass_like_the_reference():
    """cvmm.py:12-21 declares CVMMSel a @dataclass: fields(), replace() and
    asdict() work on it with the same field names and defaults."""
    import dataclasses
    s = _plain_sel()
    assert dataclasses.is_dataclass(s)
    assert [f.name for f in dataclasses.fields(C.CVMMSel)] == [
        "raw_sel", "sel", "sel_index", "out_index", "reduction_weight"]
    w = torch.rand(2, 2)
    r = dataclasses.replace(s, reduction_weight=w)
    assert isinstance(r, C.CVMMSel) and r.reduction_weight is w
    assert r.raw_sel is s.raw_sel and r.sel is s.sel and r.out_index is s.out_index
    d = dataclasses.asdict(s)
    assert list(d) == ["raw_sel", "sel", "sel_index", "out_index", "reduction_weight"]
    assert torch.equal(d["sel_index"], s.sel_index)
    s.out_index = None                                  # plain field assignment
    assert s.out_index is None


def test_shape_log_is_on_by_default():
    """The reference prints every new (x.shape, keys.shape) (cvmm.py:1778-1781)."""
    import os
    if "CVMM_LOG_SHAPES" in os.environ:
        pytest.skip("CVMM_LOG_SHAPES set in the environment")
    assert C.cvmm_log_shapes is True


def test_gate_gradient_chunks():
    """The gate gradient's token chunks (cvmm_gate_logits): powers of two,
    each at least 1024 tokens, until the [E x D] output tiles of the batched
    product fill the GPU (512 tiles of 128 x 64); one product where the
    tokens do not split evenly or are too few."""
    assert C._gate_grad_chunks(16384, 2048, 128) == 16     # the FFN stack: 32 tiles x 16
    assert C._gate_grad_chunks(4096, 512, 64) == 4         # 1024 tokens per chunk
    assert C._gate_grad_chunks(1000, 64, 16) == 1          # too few tokens
    assert C._gate_grad_chunks(16383, 2048, 128) == 1      # odd token count
    assert C._gate_grad_chunks(65536, 4096, 1024) == 1     # 512 tiles already
    for T, D, E in ((16384, 2048, 128), (8192, 1024, 64), (2048, 256, 32)):
        c = C._gate_grad_chunks(T, D, E)
        assert T % c == 0 and (c == 1 or T // c >= 1024)


def test_gate_logits_has_no_cpu_path():
    """cvmm_gate_logits, like the products, takes device tensors only."""
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        C.cvmm_gate_logits(torch.randn(4, 8), torch.randn(8, 3))
