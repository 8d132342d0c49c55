"""Module API of atlas_rnn_amd.rnn_memory against the reference's (atlas_pytorch/rnn_memory.py).

CPU-only checks: constructor arguments, parameter / buffer names and their order (so a
reference checkpoint loads with load_state_dict), gate-head initialisations, init_state
shapes, the feature map and the multi-head RMS norm against closed forms, and that the
recurrence refuses CPU tensors (the product path has no CPU implementation).
"""

import math
import warnings

import pytest
import torch

import atlas_rnn_amd as am
from atlas_rnn_amd import rnn_memory as rm

# Parameter names in registration order, read off the reference constructors
# (rnn_memory.py:181-237 for RNNMemoryCell, :482-534 for OmegaRNNMemoryCell).
TITANS_PARAMS = [
    "to_q.weight", "to_k.weight", "to_v.weight", "to_out.weight",
    "q_conv.weight", "k_conv.weight", "v_conv.weight",
    "to_lr.0.weight", "to_lr.0.bias", "to_decay.0.weight", "to_decay.0.bias",
    "to_momentum.0.weight", "to_momentum.0.bias",
    "pre_norm.weight", "q_norm.gamma", "k_norm.gamma",
]
OMEGA_EXTRA = ["to_omega_gate.0.weight", "to_omega_gate.0.bias"]


def test_titans_cell_parameter_names_and_inits():
    cell = am.RNNMemoryCell(dim=32, dim_head=16, heads=2)
    assert [n for n, _ in cell.named_parameters()] == TITANS_PARAMS
    assert [n for n, _ in cell.named_buffers()] == ["_dummy"]
    for head, bias in (("to_lr", -4.0), ("to_decay", 4.0), ("to_momentum", 2.0)):
        lin = getattr(cell, head)[0]
        assert lin.weight.shape == (2, 32) and torch.all(lin.weight == 0)
        assert torch.all(lin.bias == bias)
    assert cell.to_q.weight.shape == (32, 32) and cell.to_out.weight.shape == (32, 32)
    assert cell.q_conv.weight.shape == (32, 1, 4) and cell.q_conv.padding == (2,)
    assert cell.q_norm.gamma.shape == (2, 1, 16)


def test_omega_cell_parameter_names_and_inits():
    cell = am.OmegaRNNMemoryCell(dim=32, dim_head=16, heads=2, omega_window=4)
    names = [n for n, _ in cell.named_parameters()]
    expected = TITANS_PARAMS[:13] + OMEGA_EXTRA + TITANS_PARAMS[13:]
    assert names == expected
    assert torch.all(cell.to_omega_gate[0].bias == 0) and torch.all(cell.to_omega_gate[0].weight == 0)


def test_optional_parts_absent():
    cell = am.OmegaRNNMemoryCell(dim=16, dim_head=8, heads=2, omega_window=2, use_omega_gate=False,
                                 use_momentum=False, qk_norm=False, qkv_conv_kernel=None)
    names = [n for n, _ in cell.named_parameters()]
    assert names == ["to_q.weight", "to_k.weight", "to_v.weight", "to_out.weight", "to_lr.0.weight",
                     "to_lr.0.bias", "to_decay.0.weight", "to_decay.0.bias", "pre_norm.weight"]
    assert cell.q_conv is None and cell.to_momentum is None and cell.to_omega_gate is None


def test_tensor_map_registers_projection_buffer():
    cell = am.RNNMemoryCell(dim=16, dim_head=8, heads=2, poly_degree=2, poly_mode='tensor')
    buffers = dict(cell.named_buffers())
    assert buffers["phi.proj"].shape == (8 + 64, 8)


def test_state_dict_round_trip_between_cells():
    a = am.OmegaRNNMemoryCell(dim=16, dim_head=8, heads=2, omega_window=3)
    b = am.OmegaRNNMemoryCell(dim=16, dim_head=8, heads=2, omega_window=3)
    b.load_state_dict(a.state_dict(), strict=True)
    for (na, pa), (nb, pb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert na == nb and torch.equal(pa, pb)


def test_init_state_shapes():
    t = am.RNNMemoryCell(dim=16, dim_head=8, heads=3).init_state(2)
    assert t.seq_index == 0 and t.S.shape == (6, 8, 8) and t.Z.shape == (6, 8, 8) and t.omega_buffer is None
    o = am.OmegaRNNMemoryCell(dim=16, dim_head=8, heads=3, omega_window=5, use_momentum=False).init_state(
        2, dtype=torch.float64)
    assert o.Z is None and o.omega_buffer.shape == (6, 4, 8, 8) and o.S.dtype == torch.float64
    assert am.OmegaRNNMemoryCell(dim=16, dim_head=8, heads=1, omega_window=1).init_state(1).omega_buffer is None


def test_state_detach():
    S = torch.ones(2, 3, 3, requires_grad=True) * 2
    st = am.state_detach(am.RNNMemState(seq_index=5, S=S, Z=None, omega_buffer=S * 3))
    assert st.seq_index == 5 and not st.S.requires_grad and st.Z is None and not st.omega_buffer.requires_grad


def test_polynomial_feature_map_closed_forms():
    x = torch.tensor([[0.5, -2.0, 3.0]], dtype=torch.float64)
    assert torch.equal(am.PolynomialFeatureMap(3, 1, 'elementwise')(x), x)
    assert torch.equal(am.PolynomialFeatureMap(3, 3, 'off')(x), x)
    # sum_{i=1..3} x^i
    want = torch.tensor([[0.5 + 0.25 + 0.125, -2.0 + 4.0 - 8.0, 3.0 + 9.0 + 27.0]], dtype=torch.float64)
    assert torch.allclose(am.PolynomialFeatureMap(3, 3, 'elementwise')(x), want)
    m = am.PolynomialFeatureMap(16, 2, 'tensor')   # the tensor map runs on its kernels only
    assert m.proj.shape == (16 + 256, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(2, 16))
    assert am.PolynomialFeatureMap(3, 2, 'elementwise').fused_elementwise
    assert not am.PolynomialFeatureMap(3, 2, 'tensor').fused_elementwise


def test_multihead_rms_norm():
    norm = am.MultiheadRMSNorm(4, 2)
    x = torch.randn(3, 2, 5, 4, dtype=torch.float64)
    y = norm.double()(x)
    # unit root-mean-square per vector with gamma = 1
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(3, 2, 5, dtype=torch.float64))
    with torch.no_grad():
        norm.gamma[1].fill_(3.0)
    y = norm(x)
    assert torch.allclose(y[:, 1].pow(2).mean(-1), torch.full((3, 5), 9.0, dtype=torch.float64))


def test_rnn_memory_wrapper_selects_cell():
    assert isinstance(am.RNNMemory(dim=16, heads=2, dim_head=8).cell, am.RNNMemoryCell)
    assert isinstance(am.RNNMemory(dim=16, omega_window=2).cell, am.OmegaRNNMemoryCell)
    om = am.OmegaRNNMemory(dim=16, heads=2, dim_head=8)
    assert isinstance(om.cell, am.OmegaRNNMemoryCell)
    assert om.cell.omega_window == 4 and om.cell.use_omega_gate
    assert am.RNNMemory(dim=24).cell.dim_head == 24


def test_use_cuda_other_window_warns_and_uses_standard_path():
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        cell = am.OmegaRNNMemoryCell(dim=16, dim_head=8, omega_window=4, use_cuda=True)
    assert not cell.use_cuda and any("omega_window=16" in str(x.message) for x in w)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the CPU refusal")
def test_cells_refuse_cpu_tensors():
    for cell in (am.RNNMemoryCell(dim=16, dim_head=8, heads=2),
                 am.OmegaRNNMemoryCell(dim=16, dim_head=8, heads=2, omega_window=3)):
        with pytest.raises(RuntimeError, match="GPU"):
            cell(torch.randn(1, 5, 16))
    for fn, args in ((am.assoc_scan, (torch.rand(2, 3), torch.rand(2, 3, 4))),
                     (am.window_sum, (torch.rand(2, 3, 4), 2)),
                     (am.affine_associative_scan, (torch.rand(2, 3, 4, 4), torch.rand(2, 3, 2, 4)))):
        with pytest.raises(RuntimeError, match="GPU"):
            fn(*args)


def test_module_aliases():
    from atlas_rnn_amd import affine_scan, omega
    assert affine_scan.affine_associative_scan is am.affine_associative_scan
    assert omega.AssocScan is am.AssocScan
    assert rm._sliding_sum_along_time is not None and math.isfinite(1.0)


def test_get_cuda_status_keys():
    """atlas_omega_autograd.py:16-22: get_cuda_status() reports available / loaded_via / error; here
    the backend is libatlas_mem.so (built in-tree), loaded without touching a GPU."""
    st = am.get_cuda_status()
    assert set(st) == {"available", "loaded_via", "error"}
    assert isinstance(st["available"], bool) and isinstance(st["loaded_via"], str) and isinstance(st["error"], str)
    if st["available"]:
        assert st["loaded_via"].endswith("libatlas_mem.so") and st["error"] == ""
    else:
        assert st["loaded_via"] == "none" and st["error"]
    from atlas_rnn_amd import functional
    assert functional.get_cuda_status is am.get_cuda_status


def test_tensor_map_tables_are_kept_by_the_module_and_dropped_on_moves():
    """PolynomialFeatureMap keeps proj's symmetrised tables itself (not in a process-wide cache):
    moves and load_state_dict drop them, refresh_tables() too."""
    fm = am.PolynomialFeatureMap(16, 2, 'tensor')
    fm._tables[("sentinel",)] = object()
    fm.double()
    assert not fm._tables
    fm._tables[("sentinel",)] = object()
    fm.load_state_dict(fm.state_dict())
    assert not fm._tables
    fm._tables[("sentinel",)] = object()
    fm.refresh_tables()
    assert not fm._tables
    from atlas_rnn_amd import functional
    assert not hasattr(functional, "_SYM_CACHE")
