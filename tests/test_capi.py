"""CPU tests of the C ABI (include/pom_amd.h) and of the host-side module logic.

The library is loaded and every declared symbol is bound; argument
validation is exercised with calls that fail before anything touches a GPU
(no kernel is launched without one).
"""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pom_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pom_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from pom_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libpom_amd.so not built (python pom_amd/csrc/build.py)")
    return _lib.load()


def test_header_lists_expected_entry_points():
    names = _declared_functions()
    for n in ["pom_abi_version", "pom_last_error", "pom_agg_workspace_size", "pom_agg_fwd", "pom_agg_bwd",
              "pom_gate_workspace_size", "pom_gate_fwd", "pom_gate_bwd", "pom_gate_heads_workspace_size",
              "pom_gate_heads_fwd", "pom_gate_heads_bwd", "pom_features_workspace_size", "pom_features_fwd",
              "pom_features_bwd", "pom_transpose", "pom_gemm_plan", "pom_gemm_workspace_size", "pom_gemm"]:
        assert n in names


def test_every_declared_symbol_is_exported_and_bound(lib):
    from pom_amd import _lib
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/pom_amd.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature in pom_amd/_lib.py"
    assert lib.pom_abi_version() == _lib.ABI_VERSION


def test_workspace_sizes(lib):
    # valid shapes report a positive size; invalid ones report 0
    assert lib.pom_agg_workspace_size(1, 16, 1024, 2304, 2, 1024, 0, 0) > 0
    assert lib.pom_agg_workspace_size(1, 16, 1024, 2304, 2, 1024, 0, 1) > 0
    assert lib.pom_agg_workspace_size(1, 4, 16384, 4096, 2, 1024, 0, 1) > 0
    assert lib.pom_agg_workspace_size(1, 4, 16384, 4096, 2, 1, 0, 1) > 0       # token-causal
    assert lib.pom_agg_workspace_size(1, 16, 1024, 2304, 17, 1024, 0, 0) == 0  # degree > 16
    assert lib.pom_agg_workspace_size(1, 16, 1000, 2304, 2, 64, 0, 0) == 0     # frame_len must divide N
    assert lib.pom_agg_workspace_size(7, 16, 1024, 2304, 2, 1024, 0, 0) == 0   # bad dtype
    assert lib.pom_gate_workspace_size(1, 16, 1024, 2304, 1, 0) > 0
    assert lib.pom_gate_workspace_size(1, 16, 1024, 2304, 3, 0) == 0           # groups must divide N
    # the size depends only on the shape: larger shapes never need less
    a = lib.pom_agg_workspace_size(1, 8, 1024, 2304, 2, 1024, 0, 1)
    b = lib.pom_agg_workspace_size(1, 16, 1024, 2304, 2, 1024, 0, 1)
    assert b >= a


def _view(ptr=256, sb=0, sn=0):
    from pom_amd._lib import PomView
    return PomView(ptr, sb, sn)


def test_validation_errors_before_launch(lib):
    from pom_amd import _lib
    x = _view(256, 1024 * 64, 64)
    coeff = ctypes.c_void_p(512)
    out = ctypes.c_void_p(1024)
    ws = ctypes.c_void_p(4096)
    # empty shape
    rc = lib.pom_agg_fwd(1, 0, 0, 16, 64, 2, ctypes.byref(x), coeff, None, 0, 0, 16, None, 0, None, out, None,
                         ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID and b"empty shape" in lib.pom_last_error()
    # degree out of range
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 0, ctypes.byref(x), coeff, None, 0, 0, 16, None, 0, None, out, None,
                         ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_UNSUPPORTED
    # frame_len not dividing N
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, None, 0, 0, 5, None, 0, None, out, None,
                         ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID and b"frame_len" in lib.pom_last_error()
    # null coefficients / output
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), None, None, 0, 0, 16, None, 0, None, out, None,
                         ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, None, 0, 0, 16, None, 0, None, None, None,
                         ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID
    # workspace missing or too small
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, None, 0, 0, 16, None, 0, None, out, None,
                         None, 0, None)
    assert rc == _lib.POM_ERR_WORKSPACE
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, None, 0, 0, 16, None, 0, None, out, None,
                         ws, 16, None)
    assert rc == _lib.POM_ERR_WORKSPACE
    # masked forward without count_out; masked with frames
    mask = ctypes.c_void_p(2048)
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, mask, 16, 1, 16, None, 0, None, out, None,
                         ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, mask, 16, 1, 8, None, 0, None, out,
                         ctypes.c_void_p(4096), ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_UNSUPPORTED
    # carry with n_past < 1
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, None, 0, 0, 16, ctypes.c_void_p(8192), 0,
                         None, out, None, ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID
    # RoPE with an odd channel count
    rope = _lib.PomRope(_lib.ROPE_1D, 512, 512, None, None, 32, 16, 0, 512, 1)
    rc = lib.pom_agg_fwd(1, 0, 2, 16, 63, 2, ctypes.byref(x), coeff, None, 0, 0, 16, None, 0, ctypes.byref(rope),
                         out, None, ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID and b"even" in lib.pom_last_error()
    # gate: groups not dividing N
    rc = lib.pom_gate_fwd(1, 0, 2, 16, 64, ctypes.byref(x), None, ctypes.c_void_p(512), 3, None,
                          ctypes.byref(_view(4096, 1024, 64)), None, None)
    assert rc == _lib.POM_ERR_INVALID
    # channel-major copy: fp32 is not built, overlapping strides are rejected, token-causal has none
    sh = ctypes.byref(_view(4096, 1024, 64))
    tv = ctypes.byref(_lib.PomTView(8192, 32, 16))
    rc = lib.pom_gate_fwd(0, 0, 2, 16, 64, ctypes.byref(x), None, ctypes.c_void_p(512), 1, None, sh, tv, None)
    assert rc == _lib.POM_ERR_UNSUPPORTED and b"16-bit" in lib.pom_last_error()
    bad = ctypes.byref(_lib.PomTView(8192, 20, 16))   # stride_c < (B-1)*stride_b + N
    rc = lib.pom_gate_fwd(1, 0, 2, 16, 64, ctypes.byref(x), None, ctypes.c_void_p(512), 1, None, sh, bad, None)
    assert rc == _lib.POM_ERR_INVALID and b"overlap" in lib.pom_last_error()
    rc = lib.pom_agg_bwd(1, 0, 2, 16, 64, 2, ctypes.byref(x), coeff, None, 0, 0, None, 1, 0, None,
                         ctypes.c_void_p(2048), ctypes.byref(_view(4096, 1024, 64)), tv, ctypes.c_void_p(1024),
                         ws, 1 << 20, None)
    assert rc == _lib.POM_ERR_UNSUPPORTED and b"token-causal" in lib.pom_last_error()


def test_python_errors_without_gpu():
    import pom_amd
    m = pom_amd.PoM(16, 2, 2)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        m(torch.randn(1, 4, 16))
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        pom_amd.poly_agg_mean_hip(torch.randn(1, 4, 16), torch.randn(16, 2), 2)


def test_degree_and_mask_validation():
    import importlib
    import pom_amd
    from pom_amd import ops
    pm = importlib.import_module("pom_amd.pom")
    with pytest.raises(NotImplementedError):
        ops._check_degree(17)
    with pytest.raises(ValueError):
        ops._check_degree(0)
    with pytest.raises(ValueError):
        pm._frame_len_of(("block_causal", 5), 16)
    assert pm._frame_len_of(pom_amd.block_causal(4), 16) == 4


def test_module_parameters_match_reference_names_and_init():
    """Same parameter names, shapes and RNG draw order as pom/pom.py:180-191,
    checked against the oracle's init_params (pinned by the golden fixtures)."""
    import pom_amd
    from oracle import pom_oracle as O
    torch.manual_seed(0)
    m = pom_amd.PoM(32, 3, 2)
    torch.manual_seed(0)
    prm = O.init_params(32, 3, 2)
    names = sorted(n for n, _ in m.named_parameters())
    assert names == ["ag_proj.weight", "po_coeff", "qc_proj.weight", "se_bias"]
    assert torch.equal(m.qc_proj.weight, prm.w_qc) and torch.equal(m.po_coeff, prm.po_coeff)
    assert torch.equal(m.ag_proj.weight, prm.w_ag) and torch.equal(m.se_bias, prm.se_bias)
    mh = pom_amd.PoM(32, 2, 2, 1, 4)
    assert mh.qc_proj.weight.shape == (64 + 4, 32) and mh.se_bias.shape == (4,)
    mg = pom_amd.PoM(32, 2, 2, 4, 1, True)
    assert sorted(n for n, _ in mg.named_parameters()) == sorted(
        ["po_proj.weight", "po_proj.bias", "se_proj.weight", "se_proj.bias", "po_coeff", "ag_proj.weight",
         "ag_proj.bias"])
    r = pom_amd.PoMRoPE(32, 2, 2, rope_2d=True)
    assert sorted(n for n, _ in r.named_buffers()) == ["col_cos", "col_sin", "row_cos", "row_sin"]
    assert r.row_cos.shape == (64, 16)
    sd = r.state_dict()
    r2 = pom_amd.PoMRoPE(32, 2, 2, rope_2d=True)
    r2.load_state_dict(sd, strict=True)


def test_transpose_validation_before_launch(lib):
    from pom_amd import _lib
    src, dst = ctypes.c_void_p(256), ctypes.c_void_p(4096)
    assert lib.pom_transpose(1, -1, 4, src, 4, dst, 1, None) == _lib.POM_ERR_INVALID
    assert lib.pom_transpose(1, 4, 8, src, 4, dst, 4, None) == _lib.POM_ERR_INVALID   # ld_src < cols
    assert b"ld_src" in lib.pom_last_error()
    assert lib.pom_transpose(1, 4, 8, src, 8, dst, 2, None) == _lib.POM_ERR_INVALID   # ld_dst < rows
    assert lib.pom_transpose(1, 4, 8, None, 8, dst, 4, None) == _lib.POM_ERR_INVALID
    assert lib.pom_transpose(9, 4, 8, src, 8, dst, 4, None) == _lib.POM_ERR_INVALID   # bad dtype
    assert lib.pom_transpose(1, 4, 8, ctypes.c_void_p(257), 8, dst, 4, None) == _lib.POM_ERR_INVALID
    assert lib.pom_transpose(1, 0, 8, src, 8, dst, 0, None) == _lib.POM_OK            # empty: no launch


def test_param_dtype_validation(lib):
    from pom_amd import _lib
    x = _view(256, 1024 * 64, 64)
    rc = lib.pom_agg_fwd(1, 7, 2, 16, 64, 2, ctypes.byref(x), ctypes.c_void_p(512), None, 0, 0, 16, None, 0, None,
                         ctypes.c_void_p(1024), None, ctypes.c_void_p(4096), 1 << 20, None)
    assert rc == _lib.POM_ERR_INVALID and b"param_dtype" in lib.pom_last_error()
    rc = lib.pom_gate_fwd(1, 9, 2, 16, 64, ctypes.byref(x), ctypes.c_void_p(512), ctypes.c_void_p(512), 1, None,
                          ctypes.byref(_view(4096, 1024, 64)), None, None)
    assert rc == _lib.POM_ERR_INVALID and b"param_dtype" in lib.pom_last_error()


def test_heads_validation_before_launch(lib):
    """Per-head gating rejects bad shapes and RoPE layouts before any launch."""
    from pom_amd import _lib
    ys = ctypes.byref(_view(256, 64 * 8, 8))
    sh = ctypes.byref(_view(4096, 64 * 64, 64))
    hagg = ctypes.c_void_p(8192)
    # H must divide P
    rc = lib.pom_gate_heads_fwd(1, 1, 2, 64, 64, 7, ys, None, hagg, 1, None, sh, None, None)
    assert rc == _lib.POM_ERR_INVALID and b"divide P" in lib.pom_last_error()
    # groups must divide N
    rc = lib.pom_gate_heads_fwd(1, 1, 2, 64, 64, 8, ys, None, hagg, 5, None, sh, None, None)
    assert rc == _lib.POM_ERR_INVALID and b"groups" in lib.pom_last_error()
    # 1-D RoPE needs an even head count, 2-D a multiple of 4, tables wide enough
    pos = ctypes.c_void_p(512)
    r1 = _lib.PomRope(_lib.ROPE_1D, 1024, 2048, None, None, 4, 16, 0, pos.value, 1)
    rc = lib.pom_gate_heads_fwd(1, 1, 2, 64, 63, 7, ys, None, hagg, 1, ctypes.byref(r1), sh, None, None)
    assert rc == _lib.POM_ERR_INVALID and b"even" in lib.pom_last_error()
    r1n = _lib.PomRope(_lib.ROPE_1D, 1024, 2048, None, None, 3, 16, 0, pos.value, 1)
    rc = lib.pom_gate_heads_fwd(1, 1, 2, 64, 64, 8, ys, None, hagg, 1, ctypes.byref(r1n), sh, None, None)
    assert rc == _lib.POM_ERR_INVALID and b"narrower" in lib.pom_last_error()
    r2 = _lib.PomRope(_lib.ROPE_2D, 1024, 2048, 1024, 2048, 2, 16, 16, pos.value, 2)
    rc = lib.pom_gate_heads_fwd(1, 1, 2, 64, 60, 6, ys, None, hagg, 1, ctypes.byref(r2), sh, None, None)
    assert rc == _lib.POM_ERR_INVALID and b"divisible by 4" in lib.pom_last_error()
    # parameter dtype and a short workspace
    rc = lib.pom_gate_heads_fwd(1, 9, 2, 64, 64, 8, ys, None, hagg, 1, None, sh, None, None)
    assert rc == _lib.POM_ERR_INVALID and b"param_dtype" in lib.pom_last_error()
    need = lib.pom_gate_heads_workspace_size(1, 2, 64, 64, 8, 1)
    assert need > 0 and lib.pom_gate_heads_workspace_size(1, 2, 64, 64, 7, 1) == 0
    rc = lib.pom_gate_heads_bwd(1, 1, 2, 64, 64, 8, ys, None, hagg, 1, None, sh, ys, ctypes.c_void_p(1 << 16),
                                None, ctypes.c_void_p(1 << 20), need - 1, None)
    assert rc == _lib.POM_ERR_WORKSPACE


def test_features_validation_before_launch(lib):
    from pom_amd import _lib
    x = ctypes.byref(_view(256, 64 * 32, 32))
    out = ctypes.byref(_view(8192, 64 * 32, 32))
    rc = lib.pom_features_fwd(1, 1, 2, 64, 32, 17, x, ctypes.c_void_p(512), out, None)
    assert rc == _lib.POM_ERR_UNSUPPORTED and b"degree" in lib.pom_last_error()
    rc = lib.pom_features_fwd(1, 1, 2, 64, 32, 2, x, None, out, None)
    assert rc == _lib.POM_ERR_INVALID and b"coeff" in lib.pom_last_error()
    rc = lib.pom_features_fwd(5, 1, 2, 64, 32, 2, x, ctypes.c_void_p(512), out, None)
    assert rc == _lib.POM_ERR_INVALID
    need = lib.pom_features_workspace_size(1, 2, 64, 32, 2)
    assert need > 0 and lib.pom_features_workspace_size(1, 2, 64, 32, 0) == 0
    rc = lib.pom_features_bwd(1, 1, 2, 64, 32, 2, x, ctypes.c_void_p(512), out, out, ctypes.c_void_p(1024),
                              ctypes.c_void_p(1 << 20), need - 1, None)
    assert rc == _lib.POM_ERR_WORKSPACE


def test_noalloc_rejects_oversize_shapes_before_any_device_call(lib):
    """pom_agg_fwd_noalloc checks the shape's scratch need first: the token-causal
    C4 shape (64 MiB of forward scratch) is refused before anything else."""
    from pom_amd import _lib
    need = lib.pom_agg_workspace_size(1, 4, 16384, 4096, 2, 1, 0, 0)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    x = _view(256, 16384 * 4096, 4096)
    rc = lib.pom_agg_fwd_noalloc(1, 1, 4, 16384, 4096, 2, ctypes.byref(x), ctypes.c_void_p(512), None, 0, 0, 1,
                                 None, 0, None, ctypes.c_void_p(1024), None, None)
    assert rc == _lib.POM_ERR_WORKSPACE
    assert b"static scratch" in lib.pom_last_error()
    # every baseline configuration's forward fits
    for B, N, P, K, fl, rk in [(2, 256, 512, 2, 256, 0), (16, 1024, 2304, 2, 1024, 0), (32, 2048, 2048, 3, 2048, 0),
                               (4, 16384, 4096, 2, 1024, 0), (8, 4096, 3072, 2, 4096, 2)]:
        assert 0 < lib.pom_agg_workspace_size(1, B, N, P, K, fl, rk, 0) <= _lib.NOALLOC_SCRATCH_BYTES


def test_derived_copies_rebuilt_by_default_and_cache_opt_in(monkeypatch):
    """Parameter-derived copies are rebuilt on every call unless the cache is
    turned on; with it on, a write through .data (which leaves the version
    counter alone) is not seen until invalidate_derived()."""
    from pom_amd import _lib, ops
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    cache = {}
    p = torch.nn.Parameter(torch.zeros(4))
    make = lambda t: t.detach().clone() + 1
    assert not _lib.derived_cache_enabled()
    assert torch.equal(_lib.derived(cache, p, make), torch.ones(4))
    p.data.add_(1)                                   # no version bump
    assert torch.equal(_lib.derived(cache, p, make), torch.full((4,), 2.0))
    try:
        _lib.set_derived_cache(True)
        a = _lib.derived(cache, p, make)
        assert _lib.derived(cache, p, make) is a     # kept while unchanged
        p.data.add_(1)
        assert _lib.derived(cache, p, make) is a     # the documented .data limitation
        ops.invalidate_derived()
        b = _lib.derived(cache, p, make)
        assert torch.equal(b, torch.full((4,), 3.0))
        with torch.no_grad():
            p.add_(1)                                # bumps the version counter
        assert torch.equal(_lib.derived(cache, p, make), torch.full((4,), 4.0))
    finally:
        _lib.set_derived_cache(False)


def test_rope_table_copies_cached_with_the_cache_off(monkeypatch):
    """A bf16 RoPE table (a module buffer in a bf16 model) is converted to fp32
    once per table version, also with the parameter cache off; an in-place
    write (version bump) is seen; an fp32 contiguous table is used as is."""
    from pom_amd import _lib
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    assert not _lib.derived_cache_enabled()
    t = torch.linspace(-1, 1, 64).reshape(4, 16).to(torch.bfloat16)
    a = _lib._f32_table(t)
    assert a.dtype == torch.float32 and torch.equal(a, t.float())
    assert _lib._f32_table(t) is a
    t.mul_(2)
    b = _lib._f32_table(t)
    assert b is not a and torch.equal(b, t.float())
    f = torch.zeros(4, 16)
    assert _lib._f32_table(f) is f


def test_rope_positions_checked_on_host():
    """Host positions must lie in [-rows, rows) (the range torch's indexing of
    the tables accepts, pom/pom_rope.py:173-174); negatives are passed through
    for the kernels' p + rows lookup; an arange longer than the table raises."""
    from pom_amd import _lib
    fc, fs = torch.ones(8, 4), torch.zeros(8, 4)
    pos = torch.tensor([-8, -1, 0, 7])
    spec = _lib.RopeSpec(_lib.ROPE_1D, [fc, fs], pos)
    assert torch.equal(spec.pos, pos) and spec.pos.dtype == torch.int64
    for bad in ([8], [-9], [0, 100]):
        with pytest.raises(IndexError):
            _lib.RopeSpec(_lib.ROPE_1D, [fc, fs], torch.tensor(bad))
    with pytest.raises(IndexError):
        _lib.RopeSpec(_lib.ROPE_1D, [fc, fs], torch.arange(9), n_max=9)
    rc, rs, cc, cs = torch.ones(4, 2), torch.zeros(4, 2), torch.ones(6, 2), torch.zeros(6, 2)
    _lib.RopeSpec(_lib.ROPE_2D, [rc, rs, cc, cs], torch.tensor([[3, 5], [-4, -6]]))
    with pytest.raises(IndexError):
        _lib.RopeSpec(_lib.ROPE_2D, [rc, rs, cc, cs], torch.tensor([[4, 0]]))   # row table has 4 rows
    with pytest.raises(IndexError):
        _lib.RopeSpec(_lib.ROPE_2D, [rc, rs, cc, cs], torch.tensor([[0, 6]]))   # column table has 6 rows


def test_gemm_plan_and_validation_before_launch(lib):
    import ctypes
    from pom_amd import _lib
    t, sp = ctypes.c_int(-5), ctypes.c_int(-5)
    # config 2's six projection shapes all have a plan
    for M, N, K in ((16384, 4608, 1152), (16384, 1152, 2304), (16384, 2304, 1152), (16384, 1152, 4608),
                    (1152, 2304, 16384), (4608, 1152, 16384)):
        assert lib.pom_gemm_plan(M, N, K, 0, 0, ctypes.byref(t), ctypes.byref(sp)) == _lib.POM_OK
        assert 0 <= t.value < 6 and (1 <= sp.value <= 8 or sp.value == _lib.GEMM_STREAM_K)
        assert (lib.pom_gemm_workspace_size(M, N, K, -1, 0) > 0) == (sp.value > 1)
    # a width no tile divides (per-head W = 2368 at config 2) runs with a partial last tile; M and N must be
    # multiples of 8 and K of 64
    assert lib.pom_gemm_plan(2368, 1152, 16384, 1, 1, ctypes.byref(t), ctypes.byref(sp)) == _lib.POM_OK
    assert 0 <= t.value < 6
    assert lib.pom_gemm_plan(2364, 1152, 16384, 0, 0, ctypes.byref(t), ctypes.byref(sp)) == _lib.POM_ERR_UNSUPPORTED
    assert lib.pom_gemm_plan(2368, 1156, 16384, 0, 0, ctypes.byref(t), ctypes.byref(sp)) == _lib.POM_ERR_UNSUPPORTED
    assert lib.pom_gemm_plan(1024, 1024, 100, 0, 0, ctypes.byref(t), ctypes.byref(sp)) == _lib.POM_ERR_UNSUPPORTED
    assert lib.pom_gemm_workspace_size(1024, 1024, 4096, 5, 3) == 3 * 1024 * 1024 * 4
    assert lib.pom_gemm_workspace_size(1024, 1024, 4096, 5, 1) == 0
    # stream-K: one fp32 128 x 128 partial per (tile, workgroup) segment, at most 64 tiles + 255
    assert lib.pom_gemm_workspace_size(1024, 1024, 4096, 5, _lib.GEMM_STREAM_K) == (64 + 255) * 128 * 128 * 4
    assert lib.pom_gemm_workspace_size(1032, 1024, 4096, 5, _lib.GEMM_STREAM_K) == (72 + 255) * 128 * 128 * 4
    fake = 1 << 20   # never dereferenced: every call below fails validation before any launch
    call = lambda al, bl, M, N, K, odt, tile, splits, ws=None, wsb=0, **kw: lib.pom_gemm(
        al, bl, M, N, K, kw.get("A", fake), kw.get("lda", 1024), kw.get("B", fake), kw.get("ldb", 1024), odt,
        kw.get("C", fake), kw.get("ldc", 1024), tile, splits, ws, wsb, None)
    assert call(2, 0, 256, 256, 64, 1, 0, 1) == _lib.POM_ERR_INVALID          # layout
    assert call(0, 0, 256, 256, 64, 2, 0, 1) == _lib.POM_ERR_UNSUPPORTED      # fp16 output
    assert call(0, 0, 256, 256, 96, 1, 0, 1) == _lib.POM_ERR_UNSUPPORTED      # K % 64
    assert call(0, 0, 256, 256, 64, 1, 0, 1, A=0) == _lib.POM_ERR_INVALID     # null operand
    assert call(0, 0, 256, 256, 2048, 1, 0, 1, lda=1000) == _lib.POM_ERR_INVALID    # lda < K
    assert call(0, 0, 256, 256, 64, 1, 0, 1, lda=1028) == _lib.POM_ERR_UNSUPPORTED  # 16-byte rows
    assert call(0, 0, 196, 256, 64, 1, 0, 1) == _lib.POM_ERR_UNSUPPORTED      # M not a multiple of 8
    assert call(0, 0, 192, 256, 64, 1, 6, 1) == _lib.POM_ERR_UNSUPPORTED      # tile id
    assert call(0, 0, 256, 256, 640, 1, 0, 9) == _lib.POM_ERR_UNSUPPORTED     # too many splits
    assert call(0, 0, 256, 256, 640, 1, 0, 2) == _lib.POM_ERR_WORKSPACE       # split-K needs workspace
    # stream-K needs at least one 64-step per workgroup: 1 tile x 255 steps is too few, 256 enough
    assert call(0, 0, 256, 256, 255 * 64, 1, 0, _lib.GEMM_STREAM_K, lda=16384, ldb=16384) == _lib.POM_ERR_UNSUPPORTED
    assert b"stream-K" in lib.pom_last_error()
    assert call(0, 0, 256, 256, 256 * 64, 1, 0, _lib.GEMM_STREAM_K, lda=16384, ldb=16384) == _lib.POM_ERR_WORKSPACE
    assert b"workspace" in lib.pom_last_error()
    assert call(0, 0, 0, 256, 640, 1, 0, 2) == _lib.POM_OK                    # empty output: nothing to do


def test_blas_solution_registry_validates_without_a_device():
    """pom_blas_set_solution checks its shape and library before storing; a
    registered shape is reported by pom_blas_has_solution; the table's "tn"
    entries all have the K-contiguous form the layer issues."""
    from pom_amd import _lib, gemm_select
    lib = _lib.load()
    assert lib.pom_blas_set_solution(0, 64, 64, 64, 64, 64, _lib.BLAS_ROCBLAS, 1) == _lib.POM_ERR_INVALID
    assert lib.pom_blas_set_solution(64, 64, 64, 32, 64, 64, _lib.BLAS_ROCBLAS, 1) == _lib.POM_ERR_INVALID
    assert lib.pom_blas_set_solution(64, 64, 64, 64, 64, 64, 7, 1) == _lib.POM_ERR_INVALID
    assert lib.pom_blas_has_solution(96, 80, 72, 72, 72, 96) == 0
    assert lib.pom_blas_set_solution(96, 80, 72, 72, 72, 96, _lib.BLAS_HIPBLASLT, 5) == _lib.POM_OK
    assert lib.pom_blas_has_solution(96, 80, 72, 72, 72, 96) == 1
    entries = gemm_select.table_entries()
    lines = [ln for ln in open(gemm_select.TABLE) if ln.startswith("GemmTunableOp_BFloat16_TN,tn_")]
    assert len(entries) == sum(",Default," not in ln for ln in lines) >= 25
    for (m, n, k, lda, ldb, ldc), which, idx in entries:
        assert lda == k and ldb == k and ldc == m and which in (1, 2) and idx > 0
