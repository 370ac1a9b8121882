"""C ABI and host-side logic of libaetherkv — CPU only, no kernel launches.

Every entry point validates its arguments on the host before launching anything, so each error
path is exercised here with fake (never dereferenced) pointers.
"""
from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest
import torch

import aetherkv
import aetherkv._lib as L
from conftest import ROOT

FAKE = ctypes.c_void_p(0x10000)        # never dereferenced: validation fails or n == 0 first
FAKE_ODD = ctypes.c_void_p(0x10001)


@pytest.fixture(scope="module")
def lib():
    if not L.available():
        pytest.fail("libaetherkv.so is not built (run __graft_entry__.build())")
    return L.lib()


def header_functions():
    text = (ROOT / "include" / "aetherkv.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|int32_t|const char\*)\s+(aekv_\w+)\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported(lib):
    names = header_functions()
    assert len(names) >= 16
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(L.SYMBOLS)


def test_probe_library_exports_its_header_and_nothing_leaks_into_the_product():
    """bench.py's streaming probes live in libaetherkv_probe.so (include/aetherkv_probe.h), not in
    the product library, and reject bad arguments before enqueuing anything."""
    text = (ROOT / "include" / "aetherkv_probe.h").read_text()
    names = sorted(set(re.findall(r"^\s*int\s+(aekv_\w+)\(", text, flags=re.M)))
    assert names == ["aekv_scan_probe", "aekv_stream_probe"]
    path = L.LIB_PATH.with_name("libaetherkv_probe.so")
    if not path.exists():
        pytest.fail("libaetherkv_probe.so is not built (run __graft_entry__.build())")
    plib = ctypes.CDLL(str(path))
    for n in names:
        assert hasattr(plib, n), n
    assert "aekv_stream_probe" not in L.SYMBOLS and "aekv_scan_probe" not in L.SYMBOLS
    plib.aekv_stream_probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p]
    assert plib.aekv_stream_probe(None, -1, None, None, None) == 1
    assert plib.aekv_stream_probe(None, 0, None, None, None) == 0
    assert plib.aekv_stream_probe(None, 16, None, None, None) == 1
    assert plib.aekv_stream_probe(ctypes.c_void_p(0x10008), 16, FAKE, FAKE, None) == 1  # x not 16-byte aligned
    plib.aekv_scan_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    assert plib.aekv_scan_probe(None, None, 0, 32, None, None, None) == 0
    assert plib.aekv_scan_probe(FAKE, FAKE, 100, 32, None, FAKE, None) == 1  # not a multiple of 128 keys
    assert plib.aekv_scan_probe(FAKE, FAKE, 128, 48, None, FAKE, None) == 1  # row bytes neither 32 nor 64
    assert plib.aekv_scan_probe(None, FAKE, 128, 32, None, FAKE, None) == 1
    assert plib.aekv_scan_probe(ctypes.c_void_p(0x10008), FAKE, 128, 64, None, FAKE, None) == 1  # codes misaligned


def test_version_and_limits(lib):
    assert b"gfx950" in lib.aekv_version()
    assert lib.aekv_max_head_dim() == 512
    assert lib.aekv_max_topk() == 2048


@pytest.mark.parametrize("seed,d", [(42, 128), (42, 64), (7, 16), (0, 512)])
def test_host_diag_matches_torch_generator(lib, seed, d):
    out = np.empty(d, np.float32)
    assert lib.aekv_tq_diag(seed, d, out.ctypes.data_as(ctypes.c_void_p)) == L.OK
    g = torch.Generator()
    g.manual_seed(seed * 10007 + d)
    r = torch.rand(d, generator=g)
    np.testing.assert_array_equal(out, torch.where(r > 0.5, 1.0, -1.0).numpy())


def _err(lib):
    return lib.aekv_last_error().decode()


def test_encode_argument_errors(lib):
    rc = lib.aekv_tq_encode(FAKE, L.BF16, 4, 128, 3, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_VALUE and "bits must be 4 or 8" in _err(lib)
    rc = lib.aekv_tq_encode(FAKE, L.BF16, 4, 96, 8, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_VALUE and "power of 2" in _err(lib)
    rc = lib.aekv_tq_encode(FAKE, L.BF16, 4, 1024, 8, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_UNSUPPORTED
    rc = lib.aekv_tq_encode(FAKE, L.I32, 4, 128, 8, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_DTYPE
    rc = lib.aekv_tq_encode(FAKE_ODD, L.BF16, 4, 128, 8, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_ALIGN
    rc = lib.aekv_tq_encode(None, L.BF16, 4, 128, 8, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_VALUE
    rc = lib.aekv_tq_encode(FAKE, L.BF16, 1, 1, 4, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_VALUE and "even" in _err(lib)
    # empty input succeeds without launching anything
    assert lib.aekv_tq_encode(None, L.BF16, 0, 128, 4, None, None, None, None) == L.OK


def test_decode_and_wht_argument_errors(lib):
    assert lib.aekv_tq_decode(FAKE, FAKE, 4, 128, 5, FAKE, FAKE, L.BF16, None) == L.ERR_VALUE
    assert lib.aekv_tq_decode(FAKE, FAKE, 4, 128, 4, FAKE, FAKE, L.I64, None) == L.ERR_DTYPE
    assert lib.aekv_tq_decode(FAKE, FAKE, 4, 128, 4, FAKE, FAKE_ODD, L.BF16, None) == L.ERR_ALIGN
    assert lib.aekv_tq_decode(None, None, 0, 128, 4, None, None, L.BF16, None) == L.OK
    assert lib.aekv_wht(FAKE, L.F32, 4, 12, FAKE, None) == L.ERR_VALUE
    assert lib.aekv_wht(None, L.F32, 0, 16, None, None) == L.OK


def test_indexer_argument_errors(lib):
    ws_need = lib.aekv_csa_indexer_workspace_size(8, 16384, 256)
    assert ws_need >= 8 * 4 * 256 * 8
    rc = lib.aekv_csa_indexer_topk(FAKE, FAKE, FAKE, None, 8, 16384, 4, 64, 0, 0, FAKE, ws_need, FAKE, None, None)
    assert rc == L.ERR_VALUE and "k must be positive" in _err(lib)
    rc = lib.aekv_csa_indexer_topk(FAKE, FAKE, FAKE, None, 8, 16384, 4, 64, 4096, 0, FAKE, ws_need, FAKE, None, None)
    assert rc == L.ERR_UNSUPPORTED
    rc = lib.aekv_csa_indexer_topk(FAKE, FAKE, FAKE, None, 8, 16384, 4, 64, 256, 0, FAKE, ws_need - 1, FAKE, None, None)
    assert rc == L.ERR_WORKSPACE
    rc = lib.aekv_csa_indexer_topk(FAKE, FAKE, FAKE, None, 8, 16384, 4, 64, 256, 9, FAKE, ws_need, FAKE, None, None)
    assert rc == L.ERR_VALUE
    rc = lib.aekv_csa_indexer_topk_quant(FAKE, FAKE, FAKE, FAKE, FAKE, None, 8, 16384, 4, 64, 6, 256, 0, FAKE, ws_need,
                                         FAKE, None, None)
    assert rc == L.ERR_VALUE and "bits must be 4 or 8" in _err(lib)
    rc = lib.aekv_csa_indexer_topk_quant(FAKE, FAKE, FAKE, FAKE, FAKE, None, 8, 16384, 4, 48, 8, 256, 0, FAKE, ws_need,
                                         FAKE, None, None)
    assert rc == L.ERR_VALUE and "power of 2" in _err(lib)
    assert lib.aekv_csa_indexer_topk(None, None, None, None, 0, 10, 4, 64, 4, 0, None, 0, None, None, None) == L.OK


def test_attention_argument_errors(lib):
    rc = lib.aekv_sparse_sink_attention(FAKE, FAKE, FAKE, L.F32, FAKE, 1, L.BF16, 1, 1, 4, 128, 8, 4, 0.1, FAKE, None)
    assert rc == L.ERR_DTYPE and "int32 or int64" in _err(lib)
    rc = lib.aekv_sparse_sink_attention(FAKE, FAKE, FAKE, L.I64, FAKE, 3, L.BF16, 1, 1, 4, 128, 8, 4, 0.1, FAKE, None)
    assert rc == L.ERR_SHAPE and "sink" in _err(lib)
    rc = lib.aekv_sparse_sink_attention(FAKE, FAKE, FAKE, L.I64, FAKE, 1, L.BF16, 1, 1, 4, 1024, 8, 4, 0.1, FAKE, None)
    assert rc == L.ERR_UNSUPPORTED
    assert lib.aekv_sparse_sink_attention(None, None, None, L.I64, None, 1, L.BF16, 0, 1, 4, 128, 8, 4, 0.1, None,
                                          None) == L.OK
    assert lib.aekv_tiled_prefill_attention(FAKE, FAKE, FAKE, 1, L.BF16, 1, 1, 4, 128, 8, 0.1, 0, FAKE, None) == L.ERR_VALUE
    need = lib.aekv_quant_attention_workspace_size(64, 12, 128, 256, 128)
    assert need >= 64 * 6 * 12 * 130 * 4
    rc = lib.aekv_quant_sink_attention(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, 12, 128, 65536, 256, 128, 4, 0.1,
                                       FAKE, need - 1, FAKE, None)
    assert rc == L.ERR_WORKSPACE
    rc = lib.aekv_quant_sink_attention(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, 12, 96, 65536, 256, 128, 4, 0.1,
                                       FAKE, need, FAKE, None)
    assert rc == L.ERR_VALUE
    rc = lib.aekv_hca_compress(FAKE, FAKE, L.BF16, 2, 0, 16, FAKE, None)
    assert rc == L.ERR_SHAPE


def test_sink_attention_split_workspace(lib):
    ws = lib.aekv_sink_attention_workspace_size
    # no split: fp32 and other head dims (VALU kernel), launches that already fill the GPU
    assert ws(L.F32, 1, 1, 16, 128, 640, -1) == 0
    assert ws(L.BF16, 1, 1, 16, 64, 640, -1) == 0
    assert ws(L.F16, 1, 128, 16, 128, 8192, 64) == 0          # the report shape: 128 targets x 2 groups
    assert ws(L.BF16, 8, 1, 16, 128, 100, 100) == 0           # <= 4 groups of 32 per target
    # one target over 640 sources: 20 groups -> 5 pieces of 4; the combine's rows are (target, head)
    assert ws(L.BF16, 1, 1, 16, 128, 640, -1) == 16 * 5 * 132 * 4
    assert ws(L.BF16, 1, 1, 16, 128, 9999, 640) == 16 * 5 * 132 * 4
    # T = 256 targets x 16 heads over 8192 sources: 64 flash workgroups -> 8 pieces of 16 tiles
    assert ws(L.BF16, 1, 256, 16, 128, 8192, -1) == 256 * 16 * 8 * 132 * 4
    need = ws(L.BF16, 1, 1, 16, 128, 640, -1)
    rc = lib.aekv_tiled_prefill_attention_ws(FAKE, FAKE, FAKE, 16, L.BF16, 1, 1, 16, 128, 640, 0.1, 256, FAKE,
                                             need - 1, FAKE, None)
    assert rc == L.ERR_WORKSPACE and "workspace" in _err(lib)
    rc = lib.aekv_tiled_prefill_attention_ws(FAKE, FAKE, FAKE, 16, L.BF16, 1, 1, 16, 128, 640, 0.1, 256,
                                             ctypes.c_void_p(0x10010), need, FAKE, None)
    assert rc == L.ERR_ALIGN
    rc = lib.aekv_sparse_sink_attention_ws(FAKE, FAKE, FAKE, L.I32, FAKE, 16, L.F16, 1, 1, 16, 128, 9999, 640, 0.1,
                                           FAKE, need - 1, FAKE, None)
    assert rc == L.ERR_WORKSPACE


# ---- python surface (host validation, no device) ---------------------------------------------
def test_polarquant_rejects_bad_bits():
    with pytest.raises(ValueError, match="bits must be 4 or 8"):
        aetherkv.PolarQuant(bits=3)


def test_wht_rejects_non_power_of_two_before_device():
    with pytest.raises(ValueError, match="power of 2"):
        aetherkv._wht(torch.randn(3, 12))


def test_no_cpu_fallback():
    pq = aetherkv.PolarQuant(bits=8)
    with pytest.raises(RuntimeError, match="HIP device"):
        pq.encode(torch.randn(2, 128, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="HIP device"):
        aetherkv._wht(torch.randn(2, 16))


def test_polarquant_diag_cached_and_matches_torch():
    pq = aetherkv.PolarQuant(bits=4)
    d1 = pq._diag(128, torch.device("cpu"))
    assert pq._diag(128, torch.device("cpu")) is d1
    g = torch.Generator()
    g.manual_seed(42 * 10007 + 128)
    assert torch.equal(d1, torch.where(torch.rand(128, generator=g) > 0.5, 1.0, -1.0))


def test_sparse_wrappers_reject_cpu_tensors_like_reference():
    q = torch.randn(1, 1, 2, 8)
    kv = torch.randn(1, 4, 2, 8)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        aetherkv.sparse_sink_attention(q, kv, torch.zeros(1, 1, 2, dtype=torch.long), torch.zeros(2), 0.5)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        aetherkv.csa_indexer_topk(torch.randn(1, 2, 8), torch.randn(1, 5, 8), torch.randn(1, 2), 2)


def test_loader_environment_keys_and_consistency():
    # reference tests/test_cuda_loader.py:12-33
    env = aetherkv.cuda_build_environment()
    assert set(env) == {"torch_cuda_built", "torch_cuda_available", "cuda_home", "nvcc", "conda_target_include",
                        "conda_target_lib", "cuda_runtime_lib"}
    from aetherkv.backends import CudaSparseAttentionBackend

    backend = CudaSparseAttentionBackend()
    reason = aetherkv.cuda_extension_unavailable_reason(require_device=True)
    assert backend.available() is (reason is None)
    assert backend.availability_error() == reason
    assert backend.name() == "hip_extension"


def test_loader_returns_kernel_namespace():
    ext = aetherkv.load_aether_cuda_kernels()
    for n in ("sparse_sink_attention", "tiled_prefill_attention", "csa_indexer_topk", "hca_compress"):
        assert callable(getattr(ext, n))


def test_caller_output_buffers_are_checked_before_the_kernels():
    # out= / out_idx= buffers reach the kernels as raw pointers, so a wrong dtype, size or layout
    # must be refused on the host (the kernels would write B*k int64 / B*H*D bf16 past them)
    from aetherkv.decode import _check_out

    dev = torch.device("cpu")
    _check_out("out_idx", torch.empty(4, 8, dtype=torch.int64), torch.int64, 32, dev)  # accepted
    with pytest.raises(RuntimeError, match="out_idx must be torch.int64"):
        _check_out("out_idx", torch.empty(4, 8, dtype=torch.int32), torch.int64, 32, dev)
    with pytest.raises(RuntimeError, match="must hold 32 elements"):
        _check_out("out_idx", torch.empty(4, 7, dtype=torch.int64), torch.int64, 32, dev)
    with pytest.raises(RuntimeError, match="contiguous"):
        _check_out("out", torch.empty(8, 4, dtype=torch.bfloat16).t(), torch.bfloat16, 32, dev)
    with pytest.raises(RuntimeError, match="must be on"):
        _check_out("out", torch.empty(32, dtype=torch.bfloat16), torch.bfloat16, 32, torch.device("cuda:0"))


def test_fast_call_module_shares_the_library_and_its_checks(lib):
    # the CPython fast-call functions call the same loaded libaetherkv (one thread-local error
    # message: a failure through the fast call is read back through ctypes) and take the ctypes
    # calls' arguments as plain ints / floats / None
    from aetherkv import _fastcall

    fake = 0x10000
    rc = _fastcall.aekv_sparse_sink_attention_ws(fake, fake, fake, L.F32, fake, 1, L.BF16, 1, 1, 4, 128, 8, 4, 0.1,
                                                 None, 0, fake, None)
    assert rc == L.ERR_DTYPE and "int32 or int64" in _err(lib)
    rc = _fastcall.aekv_tiled_prefill_attention_ws(fake, fake, fake, 1, L.BF16, 1, 1, 4, 128, 8, 0.1, 0, None, 0,
                                                   fake, None)
    assert rc == L.ERR_VALUE
    need = lib.aekv_quant_attention_workspace_size(64, 12, 128, 256, 128)
    rc = _fastcall.aekv_quant_sink_attention(fake, fake, fake, fake, fake, fake, fake, 64, 12, 128, 65536, 256, 128, 4,
                                             0.1, fake, need - 1, fake, None)
    assert rc == L.ERR_WORKSPACE
    rc = _fastcall.aekv_csa_decode_quant(fake, fake, fake, fake, fake, None, 2, 100, 4, 64, 3, 16, 0, fake, fake,
                                         fake, fake, fake, fake, 12, 128, 16, 8, 0.1, fake, 1 << 30, fake, None, fake,
                                         None)
    assert rc == L.ERR_VALUE and "bits" in _err(lib)
    with pytest.raises(TypeError):
        _fastcall.aekv_quant_sink_attention(fake)
    assert L.hot("aekv_sparse_sink_attention_ws") is _fastcall.aekv_sparse_sink_attention_ws


def test_ring_prefix_views_are_recognised_and_others_are_not():
    """quant_sink_attention reads codes / scales in place when they are the first n rows of
    [B, S, .] storages (a CodeRing's data / scale views): the row stride S goes to the library with
    n_sel = n and no selection.  Anything else is copied to a compact tensor first."""
    from aetherkv.decode import _prefix_rows

    B, cap, rb = 3, 40, 64
    codes = torch.zeros(B, cap, rb, dtype=torch.uint8)
    scale3 = torch.zeros(B, cap, 1, dtype=torch.float32)
    scale2 = torch.zeros(B, cap, dtype=torch.float32)
    assert _prefix_rows(codes[:, :25], scale3[:, :25]) == cap
    assert _prefix_rows(codes[:, :25], scale2[:, :25]) == cap
    assert _prefix_rows(codes[:, :1], scale3[:, :1]) == cap
    assert _prefix_rows(codes, scale3) == cap  # the whole storage (contiguous callers copy nothing anyway)
    # rows 5..29 of every storage row work the same way: the pointers are those of row 5
    assert _prefix_rows(codes[:, 5:30], scale3[:, 5:30]) == cap
    # scales of another stride, a column slice, wrong dtype or mismatched lengths are refused
    assert _prefix_rows(codes[:, :25], torch.zeros(B, 2 * cap, 1)[:, :25]) is None
    assert _prefix_rows(codes[:, :25, :32], scale3[:, :25]) is None
    assert _prefix_rows(codes[:, :25], scale3[:, :25].to(torch.float64)) is None
    assert _prefix_rows(codes[:, :25], scale3[:, :24]) is None
    assert _prefix_rows(codes[:, ::2], scale3[:, ::2]) is None
    # batch-strided views whose row stride is not a multiple of the row are refused
    odd = torch.zeros(B * (cap * rb + 8), dtype=torch.uint8).as_strided((B, 25, rb), (cap * rb + 8, rb, 1))
    assert _prefix_rows(odd, scale3[:, :25]) is None
