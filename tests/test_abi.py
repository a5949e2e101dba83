"""The C-ABI library: it loads, exports every symbol the header declares, and
refuses bad arguments on the host before touching any device."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from flexkv_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flexkv_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(fkv_\w+)\s*\(", text, re.M)))


def test_header_matches_loader_list():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (fkv_\w+)", out))
    assert set(declared_functions()) <= exported


def test_single_hip_runtime_and_version():
    lib = _lib.load()
    assert lib.fkv_version().decode().startswith("flexkv_hip")
    assert len(_lib.hip_runtimes_loaded()) <= 1


def test_library_is_gfx950_code():
    """The device code bundled in the library targets gfx950 only."""
    blob = open(_lib.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx\w+)", blob))
    assert targets == {b"gfx950"}


def _call(**kw):
    ids = np.array([0, 1], dtype=np.int64)
    buf = np.zeros(1 << 16, dtype=np.uint8)
    base = (buf.ctypes.data + 255) & ~255   # 256-byte aligned address inside buf
    ptrs = (ctypes.c_void_p * 1)(base)
    args = dict(num_blocks=2, start_layer_id=0, num_layers=1, gids=ids.ctypes.data, ptrs=ptrs,
                gkv=4096, gblk=1024, cids=ids.ctypes.data, cpu=base, ckv=1024,
                clay=2048, cblk=2048, startoff=0, chunk=1024, stream=None, cus=-1, h2d=0,
                mode=0, mla=0)
    args.update(kw)
    lib = _lib.load()
    rc = lib.fkv_transfer_kv_blocks(*args.values())
    del buf
    return rc, _lib.last_error()


def test_host_side_rejections_need_no_device():
    rc, msg = _call(mode=3)
    assert rc == 1 and "use_ce_transfer" in msg
    rc, msg = _call(num_blocks=-1)
    assert rc == 1 and "negative" in msg
    rc, msg = _call(gids=None)
    assert rc == 1 and "null" in msg
    rc, msg = _call(chunk=0)
    assert rc == 1 and "chunk" in msg
    rc, msg = _call(ckv=-16)
    assert rc == 1 and "non-negative" in msg
    rc, msg = _call(chunk=24)
    assert rc == 1 and "multiples of 16" in msg
    neg = np.array([0, -3], dtype=np.int64)
    rc, msg = _call(cids=neg.ctypes.data)
    assert rc == 1 and "negative block id" in msg
    # empty transfers succeed without any device work
    assert _call(num_blocks=0)[0] == 0
    assert _call(num_layers=0)[0] == 0


def test_error_message_is_per_call():
    _call(mode=3)
    assert _lib.last_error()
    assert _call(num_blocks=0)[0] == 0
    assert _lib.last_error() == ""


def test_host_alloc_rejects_bad_flags():
    lib = _lib.load()
    p = ctypes.c_void_p()
    assert lib.fkv_host_alloc(ctypes.byref(p), 4096, 7) == 1
    assert "flags" in _lib.last_error()
    assert lib.fkv_host_alloc(ctypes.byref(p), 0, 0) == 1
    assert lib.fkv_host_free(None) == 0


def test_profile_counters_roundtrip():
    _lib.profile_enable(True)
    d = _lib.profile_read()
    assert d["kernel_launches"] == 0 and d["dma_copies"] == 0
    _lib.profile_enable(False)


def test_copy_engine_policy_setter_needs_no_device(monkeypatch):
    """fkv_set/get_copy_engine_policy: the default (32 MiB, kernel for
    scattered layer-wise ids), the environment variables while unset, explicit
    values over them, -2 keeps a field, bad values are refused."""
    import ctypes
    from flexkv_amd import c_ext
    lib = _lib.load()
    monkeypatch.delenv("FLEXKV_CE_MIN_BYTES", raising=False)
    monkeypatch.delenv("FLEXKV_CE_RECT_COPIES", raising=False)
    try:
        assert lib.fkv_set_copy_engine_policy(-1, -1) == 0
        assert c_ext.copy_engine_policy() == {"min_bytes": 32 << 20, "rect_copies": 0,
                                              "layerwise_scattered": "kernel"}
        monkeypatch.setenv("FLEXKV_CE_MIN_BYTES", "4096")
        monkeypatch.setenv("FLEXKV_CE_RECT_COPIES", "1")
        assert c_ext.copy_engine_policy()["min_bytes"] == 4096
        assert c_ext.copy_engine_policy()["rect_copies"] == 1
        c_ext.set_copy_engine_policy(min_bytes=7 << 20)
        assert c_ext.copy_engine_policy()["min_bytes"] == 7 << 20
        assert c_ext.copy_engine_policy()["rect_copies"] == 1     # kept, from the variable
        c_ext.set_copy_engine_policy(layerwise_scattered="kernel")
        assert c_ext.copy_engine_policy() == {"min_bytes": 7 << 20, "rect_copies": 0,
                                              "layerwise_scattered": "kernel"}
        assert lib.fkv_set_copy_engine_policy(-3, -2) != 0
        assert "min_bytes" in _lib.last_error()
        assert lib.fkv_set_copy_engine_policy(-2, 2) != 0
        assert "rect_copies" in _lib.last_error()
        assert lib.fkv_get_copy_engine_policy(None, None) != 0
        with pytest.raises(ValueError):
            c_ext.set_copy_engine_policy(min_bytes=-5)
        with pytest.raises(ValueError):
            c_ext.set_copy_engine_policy(layerwise_scattered="engines")
        mb, rc = ctypes.c_int64(), ctypes.c_int()
        assert lib.fkv_get_copy_engine_policy(ctypes.byref(mb), ctypes.byref(rc)) == 0
        assert (mb.value, rc.value) == (7 << 20, 0)
    finally:
        c_ext.set_copy_engine_policy(min_bytes="unset", layerwise_scattered="unset")


def test_tp_group_host_side_rejections_need_no_device():
    """fkv_tp_group_create / _transfer / _destroy refuse bad arguments with a
    message before any device work, and a null group is a no-op to destroy."""
    lib = _lib.load()
    out = ctypes.c_void_p()
    devs = (ctypes.c_int * 2)(0, 0)
    ptrs = (ctypes.c_void_p * 4)(16, 32, 48, 64)
    assert lib.fkv_tp_group_create(0, devs, ptrs, 2, ctypes.c_void_p(64), ctypes.byref(out)) == 1
    assert "ranks" in _lib.last_error()
    assert lib.fkv_tp_group_create(2, None, ptrs, 2, ctypes.c_void_p(64), ctypes.byref(out)) == 1
    assert "null" in _lib.last_error()
    assert lib.fkv_tp_group_create(2, devs, ptrs, 2, ctypes.c_void_p(64), None) == 1
    assert out.value is None
    ids = np.zeros(1, dtype=np.int64)
    rc = lib.fkv_tp_group_transfer(None, 1, ids.ctypes.data, 0, 0, 16, ids.ctypes.data, 0, 0, 0,
                                   -1, 0, 0, 0, 1, 0)
    assert rc == 1 and "null TP group" in _lib.last_error()
    assert lib.fkv_tp_group_destroy(None) == 0
