"""C-ABI checks that need no GPU: the library loads, exports every symbol include/atlas_mem.h
declares, and validates problems / sizes buffers on the host."""

import ctypes
import os
import re

import pytest

from atlas_rnn_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "atlas_mem.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(atlas_\w+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libatlas_mem.so is not built (run `python -m atlas_rnn_amd.build`)")
    return _lib.load()


def test_header_and_binding_agree():
    assert _declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.atlas_mem_abi_version() == _lib.ABI_VERSION
    assert "#define ATLAS_MEM_ABI_VERSION 1" in open(HEADER).read()


def _prob(**kw):
    p = _lib.Problem(abi_version=_lib.ABI_VERSION, bh=32, seq_len=4096, d_k=64, d_v=64, window=4, momentum=1,
                     gate_mode=_lib.GATE_LAG, map_mode=0, map_degree=1, has_buffer=0, clamp_every=0,
                     clamp_final=1, dtype=_lib.DT_BF16)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_validate_accepts_headline(lib):
    assert lib.atlas_mem_validate(ctypes.byref(_prob())) == _lib.OK


@pytest.mark.parametrize("field,value,code", [
    ("abi_version", 2, 1), ("bh", 0, 2), ("seq_len", 0, 2), ("d_k", 48, 2), ("d_v", 32, 2),
    ("window", 0, 2), ("window", 34, 2), ("dtype", 7, 3), ("momentum", 2, 9), ("gate_mode", 3, 9),
    ("map_mode", 2, 9), ("map_degree", 0, 9), ("clamp_every", -1, 9)])
def test_validate_rejects(lib, field, value, code):
    assert lib.atlas_mem_validate(ctypes.byref(_prob(**{field: value}))) == code
    assert lib.atlas_mem_saved_bytes(ctypes.byref(_prob(**{field: value}))) == 0


def test_buffer_needs_window(lib):
    assert lib.atlas_mem_validate(ctypes.byref(_prob(window=1, has_buffer=1))) == 9


def test_window_longer_than_clamp_chunk_is_unsupported(lib):
    # clamp every 4 tokens with window 8: the caller splits the call (reference chunk loop)
    assert lib.atlas_mem_validate(ctypes.byref(_prob(window=8, clamp_every=4))) == _lib.ERR_UNSUPPORTED


@pytest.mark.parametrize("every", [37, 41, 47, 53, 59, 61, 74])
def test_clamp_every_without_a_usable_chunk_is_split_by_the_caller(lib, every):
    # no divisor >= 8 usable as a chunk: the library refuses (the host splits the call at
    # clamp_every) instead of walking 1-token chunks with a state saved after each token
    p = _prob(clamp_every=every)
    assert lib.atlas_mem_validate(ctypes.byref(p)) == _lib.ERR_UNSUPPORTED
    assert lib.atlas_mem_saved_bytes(ctypes.byref(p)) == 0


@pytest.mark.parametrize("every", [32, 48, 64, 96, 100, 128])
def test_clamp_every_saved_bytes_stay_bounded(lib, every):
    # usable clamp chunks keep the saved states at backward-chunk granularity (<= 1 per 8 tokens)
    st = 64 * 64 * 4
    p = _prob(clamp_every=every)
    assert lib.atlas_mem_validate(ctypes.byref(p)) == 0
    assert lib.atlas_mem_saved_bytes(ctypes.byref(p)) <= 32 * (4096 // 8) * 2 * st + 64 * 2 ** 20


def test_sizes(lib):
    p = _prob()
    st = 64 * 64 * 4
    saved = lib.atlas_mem_saved_bytes(ctypes.byref(p))
    # bf16, d = 64, no clamp: the backward of chunk_bwd.hip reads the chunk-start (S, Z) in bf16 at
    # every 64-token boundary and forms its own records: at least those states, less than the raw
    # (S, Z) at every 32-token boundary that the other backward reads
    assert 32 * (4096 // 64) * 64 * 64 * 2 * 2 <= saved < 32 * (4096 // 32) * 2 * st
    assert saved % 256 == 0
    ws = lib.atlas_mem_bwd_workspace_bytes(ctypes.byref(p))
    assert ws > 0 and ws % 256 == 0
    # a carried buffer takes the other backward: boundary states saved
    pb = _prob(has_buffer=1)
    assert lib.atlas_mem_saved_bytes(ctypes.byref(pb)) >= 32 * (4096 // 32) * 2 * st + 32 * st
    pf = _prob(dtype=_lib.DT_F32)   # fp32: 16-token backward chunks
    assert lib.atlas_mem_saved_bytes(ctypes.byref(pf)) >= 32 * (4096 // 16) * 2 * st
    # clamping every 32 tokens forbids folding across clamps: one segment per row
    pc = _prob(clamp_every=32)
    assert lib.atlas_mem_validate(ctypes.byref(pc)) == 0
    assert lib.atlas_mem_saved_bytes(ctypes.byref(pc)) >= 32 * (4096 // 32) * 2 * st


def test_noalloc_backward_host_checks(lib):
    # the static scratch is 64 MiB: the headline shapes fit, a larger workspace is refused before any
    # HIP call, as are missing pointers
    assert lib.atlas_mem_noalloc_scratch_bytes() == 64 << 20
    assert lib.atlas_mem_bwd_workspace_bytes(ctypes.byref(_prob())) <= 64 << 20          # C3
    assert lib.atlas_mem_bwd_workspace_bytes(ctypes.byref(_prob(bh=64, seq_len=2048, gate_mode=_lib.GATE_TOKEN))) <= 64 << 20
    good = ctypes.c_void_p(0x10000)
    args = _lib.BwdArgs()
    big = _prob(bh=4096)
    assert lib.atlas_mem_bwd_workspace_bytes(ctypes.byref(big)) > 64 << 20
    assert lib.atlas_mem_bwd_noalloc(ctypes.byref(big), ctypes.byref(args), good, None) == _lib.ERR_SCRATCH
    assert lib.atlas_mem_bwd_noalloc(ctypes.byref(_prob()), None, good, None) == 4
    assert lib.atlas_mem_bwd_noalloc(ctypes.byref(_prob()), ctypes.byref(args), None, None) == 4
    assert lib.atlas_mem_bwd_noalloc(ctypes.byref(_prob(d_k=48)), ctypes.byref(args), good, None) == 2
    assert b"64 MiB" in lib.atlas_mem_strerror(_lib.ERR_SCRATCH)


def test_affine_scan_host_checks(lib):
    good = ctypes.c_void_p(0x10000)
    assert lib.atlas_affine_scan_workspace_bytes(2, 1024, 64, 64) > 0
    assert lib.atlas_affine_scan_workspace_bytes(2, 1024, 65, 64) == 0
    assert lib.atlas_affine_scan_fwd(2, 16, 8, 8, good, good, None, good, None, 0, None) == 4       # no workspace
    ws = lib.atlas_affine_scan_workspace_bytes(2, 16, 8, 8)
    assert lib.atlas_affine_scan_fwd(2, 16, 8, 8, good, good, None, good, good, ws - 1, None) == 7  # too small
    assert lib.atlas_affine_scan_fwd(2, 16, 8, 8, ctypes.c_void_p(0x10002), good, None, good, good, ws, None) == 5
    assert lib.atlas_affine_scan_bwd(2, 16, 70, 8, good, good, None, good, good, good, None, good, ws, None) == 2


def test_strerror(lib):
    for code in range(0, 11):
        assert len(lib.atlas_mem_strerror(code)) > 0
    assert b"unknown" in lib.atlas_mem_strerror(99)


def test_null_pointer_errors_before_launch(lib):
    p = _prob()
    args = _lib.FwdArgs()
    assert lib.atlas_mem_fwd(ctypes.byref(p), ctypes.byref(args), None, None) == 4
    assert lib.atlas_mem_fwd(ctypes.byref(p), None, None, None) == 4
    bargs = _lib.BwdArgs()
    assert lib.atlas_mem_bwd(ctypes.byref(p), ctypes.byref(bargs), None, None, 0, None) == 4
    assert lib.atlas_scan_fwd(0, 1, 4, 8, None, None, None, None, None) == 4
    assert lib.atlas_scan_fwd(0, 0, 4, 8, None, None, None, None, None) == 2
    assert lib.atlas_window_sum(0, 1, 4, 8, 0, 0, None, None, None) == 2


def test_misaligned_pointers_error_before_launch(lib):
    # validation happens before any HIP call: the (never dereferenced) addresses only have to be
    # non-null; a pointer off a 16-byte boundary is rejected with ERR_ALIGN
    p = _prob()
    good, bad = 0x10000, 0x10008
    fields = dict(k=good, q=good, v=good, lr=good, decay=good, beta=good, gate=good, S_ref=good, S0=good,
                  Z0=good, y=good, S_T=good, Z_T=good, buffer_out=good)
    for name in ("k", "lr", "S_ref", "S0", "buffer_out"):
        f = dict(fields, **{name: bad})
        args = _lib.FwdArgs(**{k: ctypes.c_void_p(v) for k, v in f.items()})
        assert lib.atlas_mem_fwd(ctypes.byref(p), ctypes.byref(args), ctypes.c_void_p(good), None) == 5, name
    args = _lib.FwdArgs(**{k: ctypes.c_void_p(v) for k, v in fields.items()})
    assert lib.atlas_mem_fwd(ctypes.byref(p), ctypes.byref(args), ctypes.c_void_p(bad), None) == 5


def test_step_errors_before_launch(lib):
    # atlas_mem_step: one token only; null, inconsistent and misaligned arguments are rejected
    # before any HIP call
    good, bad = 0x10000, 0x10008
    fields = dict(k=good, q=good, v=good, lr=good, decay=good, beta=good, gate=good, S_ref=good, S0=good,
                  Z0=good, y=good, S_T=good, Z_T=good, buffer_out=good)
    args = _lib.FwdArgs(**{k: ctypes.c_void_p(v) for k, v in fields.items()})
    assert lib.atlas_mem_step(ctypes.byref(_prob(seq_len=4096)), ctypes.byref(args), None) == 2
    assert lib.atlas_mem_step(ctypes.byref(_prob(seq_len=1)), None, None) == 4
    assert lib.atlas_mem_step(None, ctypes.byref(args), None) == 4
    assert lib.atlas_mem_step(ctypes.byref(_prob(seq_len=1)), ctypes.byref(_lib.FwdArgs()), None) == 4
    assert lib.atlas_mem_step(ctypes.byref(_prob(seq_len=1, momentum=0)), ctypes.byref(args), None) == 9
    assert lib.atlas_mem_step(ctypes.byref(_prob(seq_len=1, d_k=48)), ctypes.byref(args), None) == 2
    for name in ("k", "gate", "S0", "buffer_out"):
        a = _lib.FwdArgs(**{k: ctypes.c_void_p(v) for k, v in dict(fields, **{name: bad}).items()})
        assert lib.atlas_mem_step(ctypes.byref(_prob(seq_len=1)), ctypes.byref(a), None) == 5, name


def test_factored_buffer_errors_before_launch(lib):
    # atlas_mem_step_factored / atlas_buffer_factors / atlas_buffer_expand: null, inconsistent,
    # overlapping and misaligned arguments are rejected before any HIP call
    good, bad = 0x10000, 0x10008
    fields = dict(k=good, q=good, v=good, lr=good, decay=good, beta=good, gate=good, S_ref=good, S0=good,
                  Z0=good, y=good, S_T=good, Z_T=good)
    args = _lib.FwdArgs(**{k: ctypes.c_void_p(v) for k, v in fields.items()})
    st = lib.atlas_mem_step_factored
    p1 = _prob(seq_len=1, has_buffer=1)           # window 4, d 64, bh 32
    f_in, f_out = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x200000)
    assert st(ctypes.byref(_prob(seq_len=2)), ctypes.byref(args), f_in, f_out, None) == 2
    assert st(ctypes.byref(p1), ctypes.byref(args), None, f_out, None) == 4          # has_buffer needs factors_in
    assert st(ctypes.byref(p1), ctypes.byref(args), f_in, None, None) == 4           # window > 1 needs factors_out
    assert st(ctypes.byref(p1), ctypes.byref(args), f_in, ctypes.c_void_p(0x100000 + 4096), None) == 9   # overlap
    assert st(ctypes.byref(p1), ctypes.byref(args), ctypes.c_void_p(bad), f_out, None) == 5
    dense = _lib.FwdArgs(**{k: ctypes.c_void_p(v) for k, v in dict(fields, buffer_out=good).items()})
    assert st(ctypes.byref(p1), ctypes.byref(dense), f_in, f_out, None) == 9          # no dense buffer here
    bf = lib.atlas_buffer_factors
    k = ctypes.c_void_p(good)
    assert bf(ctypes.byref(_prob(window=1, has_buffer=0)), k, k, None, k, None, f_out, None) == 2
    pb = _prob(has_buffer=1)
    assert bf(ctypes.byref(pb), k, k, k, k, None, f_out, None) == 4                    # has_buffer needs factors_in
    assert bf(ctypes.byref(pb), k, k, None, k, f_in, f_out, None) == 9                 # lag gates need the gate
    assert bf(ctypes.byref(pb), k, k, k, k, f_in, f_in, None) == 9                     # in place
    ex = lib.atlas_buffer_expand
    assert ex(0, 3, 64, 64, k, k, None) == 2
    assert ex(2, 0, 64, 64, None, None, None) == 0                                    # nothing to expand
    assert ex(2, 3, 64, 64, None, k, None) == 4
    assert ex(2, 3, 64, 64, k, ctypes.c_void_p(bad), None) == 5


def test_tensor_map_errors_before_launch(lib):
    good, bad = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x10008)
    f = lib.atlas_tensor_map_fwd
    b = lib.atlas_tensor_map_bwd
    assert f(2, 8, 64, 128, 1, good, good, good, None, None) == 3                   # bf16 or fp32
    assert f(_lib.DT_F32, 8, 48, 128, 1, good, good, good, None, None) == 2         # d_in in (16, 32, 64)
    assert f(_lib.DT_BF16, 8, 128, 128, 1, good, good, good, None, None) == 2
    assert f(_lib.DT_BF16, 8, 64, 72, 1, good, good, good, None, None) == 2         # d_out % 16 == 0
    assert f(_lib.DT_F32, 8, 64, 144, 1, good, good, good, None, None) == 2         # d_out <= 128
    assert f(_lib.DT_F32, 8, 16, 16, 1, good, bad, good, None, None) == 5
    assert f(_lib.DT_BF16, 8, 64, 128, 0, good, good, good, None, None) == 2        # degree 1..16
    assert f(_lib.DT_BF16, 8, 64, 128, 1, None, good, good, None, None) == 4
    assert f(_lib.DT_BF16, 8, 64, 128, 3, good, good, good, None, None) == 4        # degree > 1 needs pre
    assert f(_lib.DT_BF16, 8, 64, 128, 1, good, bad, good, None, None) == 5
    assert f(_lib.DT_BF16, 0, 64, 128, 1, good, good, good, None, None) == 0        # empty: nothing launched
    assert b(_lib.DT_BF16, 8, 64, 128, 1, good, good, None, good, None, None) == 4
    assert b(_lib.DT_BF16, 8, 64, 128, 1, good, good, None, bad, good, None) == 5
    assert b(_lib.DT_BF16, 8, 64, 128, 2, good, good, None, good, good, None) == 4  # degree > 1 needs pre
    assert b(_lib.DT_BF16, -1, 64, 128, 1, good, good, None, good, good, None) == 2
    sy = lib.atlas_tensor_map_symmetrize
    fs = lib.atlas_tensor_map_fwd_sym
    assert sy(2, 64, 128, good, good, good, None) == 3
    assert sy(_lib.DT_BF16, 48, 128, good, good, good, None) == 2
    assert sy(_lib.DT_BF16, 64, 72, good, good, good, None) == 2
    assert sy(_lib.DT_BF16, 64, 128, good, None, good, None) == 4
    assert sy(_lib.DT_F32, 64, 128, good, good, bad, None) == 5
    assert fs(_lib.DT_BF16, 8, 64, 128, 3, good, good, good, None, None) == 4       # degree > 1 needs pre
    assert fs(_lib.DT_BF16, 8, 64, 128, 1, good, bad, good, None, None) == 5
    assert fs(_lib.DT_BF16, 8, 64, 136, 1, good, good, good, None, None) == 2
    assert fs(_lib.DT_F32, 8, 48, 128, 1, good, good, good, None, None) == 2         # fp32 takes the plain checks
    assert fs(_lib.DT_BF16, 0, 64, 128, 1, good, good, good, None, None) == 0
    bs = lib.atlas_tensor_map_bwd_sym
    assert bs(_lib.DT_BF16, 8, 64, 128, 1, good, good, None, good, None, None) == 4
    assert bs(_lib.DT_BF16, 8, 64, 128, 1, good, good, None, bad, good, None) == 5
    assert bs(_lib.DT_BF16, 8, 64, 128, 2, good, good, None, good, good, None) == 4   # degree > 1 needs pre
    assert bs(_lib.DT_BF16, 8, 64, 136, 1, good, good, None, good, good, None) == 2
    assert bs(_lib.DT_F32, 8, 48, 128, 1, good, good, None, good, good, None) == 2     # fp32 takes the plain checks
    assert bs(_lib.DT_BF16, 0, 64, 128, 1, good, good, None, good, good, None) == 0


def test_linear_wgrad_errors_before_launch(lib):
    good, bad = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x10008)
    ws = lib.atlas_linear_wgrad_workspace_bytes
    g = lib.atlas_linear_wgrad
    assert ws(16384, 512, 512) == 16 * 16 * 128 * 128 * 4          # 16 token splits x 16 tiles of 128 x 128
    assert ws(1000, 32, 512) == 4 * 4 * 128 * 128 * 4              # 256-token splits on 4 tiles
    assert ws(0, 512, 512) == 0
    assert ws(100, 12, 512) == -1 and ws(-1, 64, 64) == -1           # features % 8 == 0; n >= 0
    need = ws(1000, 32, 512)
    assert g(2, 1000, 32, 512, good, good, good, good, need, None) == 3          # dW bf16 or fp32
    assert g(_lib.DT_BF16, 1000, 36, 512, good, good, good, good, need, None) == 2
    assert g(_lib.DT_BF16, 1000, 32, 512, None, good, good, good, need, None) == 4
    assert g(_lib.DT_BF16, 1000, 32, 512, good, good, good, None, need, None) == 4   # n > 0 needs workspace
    assert g(_lib.DT_BF16, 1000, 32, 512, good, bad, good, good, need, None) == 5
    assert g(_lib.DT_F32, 1000, 32, 512, good, good, good, good, need - 4, None) == 7
    I32, VP = ctypes.c_int * 2, ctypes.c_void_p * 2
    bws = lib.atlas_linear_wgrad_batch_workspace_bytes
    gb = lib.atlas_linear_wgrad_batch
    # a batch shares the token splits: 16384 tokens over 16 + 4 tiles -> 25 splits of 672 tokens
    assert bws(2, 16384, I32(512, 32), I32(512, 512)) == 25 * (16 + 4) * 128 * 128 * 4
    assert bws(0, 100, I32(8, 8), I32(8, 8)) == -1 and bws(5, 100, I32(8, 8), I32(8, 8)) == -1
    need2 = bws(2, 1000, I32(64, 32), I32(64, 512))
    assert gb(_lib.DT_BF16, 2, 1000, I32(64, 36), I32(64, 512), VP(good, good), VP(good, good), VP(good, good),
              good, need2, None) == 2
    assert gb(_lib.DT_BF16, 2, 1000, I32(64, 32), I32(64, 512), VP(good, None), VP(good, good), VP(good, good),
              good, need2, None) == 4
    assert gb(_lib.DT_BF16, 2, 1000, I32(64, 32), I32(64, 512), VP(good, good), VP(good, bad.value), VP(good, good),
              good, need2, None) == 5
    assert gb(_lib.DT_BF16, 2, 1000, I32(64, 32), I32(64, 512), VP(good, good), VP(good, good), VP(good, good),
              good, need2 - 4, None) == 7


def test_tensor_feature_map_raises_off_kernel():
    """The map has one implementation, the kernels: CPU tensors and operands they do not take raise
    before anything is launched (no tensor-op formulation to fall back to)."""
    torch = pytest.importorskip("torch")
    from atlas_rnn_amd.functional import tensor_feature_map
    x = torch.randn(5, 7, 16)
    P = torch.randn(16 + 256, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        tensor_feature_map(x, P)
    with pytest.raises(TypeError, match="dtype"):
        tensor_feature_map(x.double(), P.double())
    with pytest.raises(ValueError, match="d_in"):
        tensor_feature_map(torch.randn(3, 24), torch.randn(24 + 576, 16))
    with pytest.raises(ValueError, match="d_out"):
        tensor_feature_map(x, torch.randn(16 + 256, 24))
    with pytest.raises(ValueError, match="proj"):
        tensor_feature_map(x, torch.randn(16 + 255, 16))
    with pytest.raises(NotImplementedError, match="constant"):
        tensor_feature_map(x, P.requires_grad_(True))
    with pytest.raises(ValueError, match="degree"):
        tensor_feature_map(x, P.detach(), degree=0)


def test_cpu_tensors_are_rejected():
    torch = pytest.importorskip("torch")
    from atlas_rnn_amd.functional import memory_recurrence
    x = torch.zeros(1, 4, 32)
    s = torch.zeros(1, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        memory_recurrence(x, x, x, s, s)


def test_linear_batch_errors_before_launch(lib):
    good, bad = 0x10000, 0x10008
    I32, VP = ctypes.c_int * 2, ctypes.c_void_p * 2
    f = lib.atlas_linear_batch
    ok = dict(n=I32(64, 32), k=I32(64, 64), a=VP(good, good), b=VP(good, good), c=VP(good, good))
    call = lambda layout=0, count=2, m=100, **kw: f(layout, count, m, *[kw.get(x, ok[x]) for x in ("n", "k", "a", "b", "c")],
                                                    None)
    assert call(layout=2) == 9                                   # NT or NN
    assert call(count=0) == 2 and call(count=5) == 2              # one to four problems
    assert call(n=I32(64, 36)) == 2 and call(k=I32(4, 64)) == 2   # multiples of 8
    assert call(m=-1) == 2
    assert call(a=VP(good, None)) == 4
    assert call(c=VP(good, bad)) == 5
    assert call(m=0, a=VP(None, None), c=VP(None, None)) == 0    # m = 0: nothing launched


def test_partials_sum_errors_before_launch(lib):
    good = 0x10000
    I32, VP = ctypes.c_int * 2, ctypes.c_void_p * 2
    f = lib.atlas_partials_sum
    assert f(0, 4, I32(8, 8), VP(good, good), VP(good, good), I32(1, 1), None) == 2      # one to eight arrays
    assert f(9, 4, I32(8, 8), VP(good, good), VP(good, good), I32(1, 1), None) == 2
    assert f(2, -1, I32(8, 8), VP(good, good), VP(good, good), I32(1, 1), None) == 2
    assert f(2, 4, I32(8, 0), VP(good, good), VP(good, good), I32(1, 1), None) == 2
    assert f(2, 4, I32(8, 8), VP(good, good), VP(good, good), I32(1, 2), None) == 3      # bf16 or fp32 out
    assert f(2, 4, I32(8, 8), VP(good, None), VP(good, good), I32(1, 0), None) == 4
    assert f(2, 4, I32(8, 8), VP(good, good), VP(None, good), I32(1, 0), None) == 4


def test_replicas_errors_before_launch(lib):
    good, odd = 0x10000, 0x10001
    I64, VP = ctypes.c_int64 * 2, ctypes.c_void_p * 2
    f = lib.atlas_replicas
    assert f(2, 1, 2, 2, I64(8, 8), VP(good, good), VP(good, good), None) == 9        # op
    assert f(0, 2, 2, 2, I64(8, 8), VP(good, good), VP(good, good), None) == 3                      # dtype
    assert f(0, 1, 0, 2, I64(8, 8), VP(good, good), VP(good, good), None) == 2                      # 1-4 arrays
    assert f(0, 1, 5, 2, I64(8, 8), VP(good, good), VP(good, good), None) == 2
    assert f(1, 1, 2, 0, I64(8, 8), VP(good, good), VP(good, good), None) == 2                      # 1-64 replicas
    assert f(1, 1, 2, 65, I64(8, 8), VP(good, good), VP(good, good), None) == 2
    assert f(0, 1, 2, 2, I64(8, -1), VP(good, good), VP(good, good), None) == 2
    assert f(0, 1, 2, 2, I64(8, 8), VP(good, None), VP(good, good), None) == 4
    assert f(0, 1, 2, 2, None, VP(good, good), VP(good, good), None) == 4
    assert f(0, 1, 2, 2, I64(8, 8), VP(good, odd), VP(good, good), None) == 5                     # element alignment
    assert f(0, 1, 2, 2, I64(0, 0), VP(None, None), VP(None, None), None) == 0                    # nothing to do
