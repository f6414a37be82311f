"""The C-ABI library loads and exports every symbol include/bc2n.h declares
(no GPU work: only load, lookup and pure-host calls)."""
import ctypes
import os

import pytest

import bindcraft2_amd as b


def test_library_exports_header_symbols():
    if not os.path.exists(b.LIB_PATH):
        pytest.fail(f"{b.LIB_PATH} not built; run __graft_entry__.build()")
    L = ctypes.CDLL(b.LIB_PATH)
    names = b.exported_symbols()
    assert len(names) >= 8
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_host_only_calls():
    L = b.lib()
    assert L.bc2n_abi_version() >= 1
    assert L.bc2n_last_error() == b""
    # save-set sizes are pure host arithmetic
    assert L.bc2n_triattn_save_bytes(64, 128, 4) > 64 * 64 * 128


def test_bad_arguments_return_status_not_exit():
    L = b.lib()
    st = L.bc2n_dropout_table(None, None, 4, 4, 0, 0, 0.25)
    assert st != 0
    assert b"bad table shape" in L.bc2n_last_error()
    st = L.bc2n_triattn_fwd(None, None, None, 0, 32, None, None, None, None, None)
    assert st != 0
    assert b"weights_dir" in L.bc2n_last_error()


def test_noalloc_refuses_weights_not_resident():
    # host-side refusal: the weights cache is consulted before any GPU call
    L = b.lib()
    st = L.bc2n_triattn_fwd_noalloc(None, b"/nonexistent", b"p/", 0, 32, 1, 1, None, 2, 3)
    assert st != 0
    assert b"not resident" in L.bc2n_last_error()
