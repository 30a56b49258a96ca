"""CPU-side checks of the native boundary (no GPU needed).

* libmoc.so loads and exports every function include/moc.h declares.
* The ctypes signature table covers exactly the declared functions.
* Argument validation happens on the host before any launch (no device
  memory is touched: null pointers / bad shapes are rejected first).
"""

import ctypes
import os

import pytest

from memory_amd import _lib


@pytest.fixture(scope="module")
def libpath():
    if not os.path.exists(_lib.LIB_PATH):
        from memory_amd import build
        build.build()
    return _lib.LIB_PATH


def test_library_exports_every_declared_symbol(libpath):
    raw = ctypes.CDLL(libpath)
    names = _lib.declared_symbols()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(raw, n)]
    assert not missing, f"declared in include/moc.h but not exported: {missing}"


def test_signature_table_matches_header():
    assert set(_lib.declared_symbols()) == set(_lib._SIGS)


def test_abi_version(libpath):
    assert _lib.lib().moc_abi_version() == 1


def test_host_validation_rejects_before_launch(libpath):
    # null pointers / bad shapes are caught on the host: no HIP call is made.
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("moc_router_topk", None, 4, 10, 1, 3, None, None, None, None)
    with pytest.raises(ValueError, match="exclude_prefix_chapters"):
        _lib.call("moc_router_topk", 1, 4, 10, 11, 3, 1, 1, None, None)
    with pytest.raises(ValueError, match="k=20"):
        _lib.call("moc_router_topk", 1, 4, 10, 1, 20, 1, 1, None, None)
    with pytest.raises(ValueError, match="head_dim 64"):
        _lib.call("moc_xattn_fwd", _lib.MOC_BF16, 1, 1, 1, 4096, 4096, 4096, 64, 1, 1, 2, 8, 4, 4, 32, 64, 5, 0.1, 1,
                  1, None)
    with pytest.raises(ValueError, match="row stride >= 64"):
        _lib.call("moc_xattn_fwd", _lib.MOC_BF16, 1, 1, 1, 4096, 4096, 4096, 32, 1, 1, 2, 8, 4, 4, 64, 64, 5, 0.1, 1,
                  1, None)
    with pytest.raises(ValueError, match="multiple of 64"):
        _lib.call("moc_kv_project", _lib.MOC_BF16, 1, _lib.MOC_BF16, 100, 64, 1, 1, 4, None, None, 1, 4, 64, 1, 1,
                  None, None, None)
    with pytest.raises(ValueError, match="C=20000"):
        _lib.call("moc_chapter_plan", 1, 10, 20000, 1, 1 << 30, 1, 1, 1, 1, 1, None)
    assert "C=20000" in _lib.lib().moc_last_error().decode()


def test_workspace_queries(libpath):
    assert _lib.query("moc_chapter_plan_workspace", 520, 4097) == (1 * 4097 + 3 * 4097) * 4
    assert _lib.query("moc_router_pool_workspace", 8, 1024, 768) == 64 * 8 * 768 * 4  # 16 rows per split
    assert _lib.query("moc_router_linear_bwd_workspace", 8, 768, 4097) == 257 * 8 * 768 * 4  # 16 chapters / wg


def test_cpu_tensors_are_rejected():
    import torch
    from memory_amd import ops
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ops.router_topk(torch.randn(2, 10), 3, 1)


def test_seq_layer_stage_names(libpath):
    """The native layer's timed stages carry distinct names, and the stages the benchmark maps to
    algorithmic work (the attention kernels, the chapter GEMMs) are among them."""
    names = _lib.seq_stage_names()
    assert len(names) == len(set(names)) >= 20
    for n in ("moc_xattn_fwd", "moc_xattn_bwd_dq", "moc_xattn_bwd_dkv", "moc_chapter_project", "moc_chapter_wgrad",
              "moc_chapter_dx", "moc_rows_linear:q_proj", "moc_rows_linear:o_proj"):
        assert n in names
    assert _lib.lib().moc_seq_layer_stage_name(len(names)) is None
    with pytest.raises(ValueError):
        _lib.seq_stage_timing(["no_such_stage"], 4)
