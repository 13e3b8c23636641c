"""libsvl.so loads and exports every function include/*.h declares; host-side validation
that needs no GPU (configuration errors are reported before any device call)."""
import ctypes as C
import os
import re

import pytest

import svl
from svl import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            text = open(os.path.join(ROOT, "include", h)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(svl_[a-z_0-9]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_binding_surface():
    assert declared_functions() == sorted(svl.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(svl.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_oracle_library_loads():
    import oracle

    L = oracle.lib()
    for name in ["svlo_model_create", "svlo_stt_step", "svlo_quantize_q8_0", "svlo_attention"]:
        assert hasattr(L, name)


@pytest.mark.parametrize("field,value,code", [
    ("num_kv_heads", 3, svl.ERR_CONFIG),       # heads not a multiple of the KV heads
    ("context", -1, svl.ERR_CONFIG),
    ("kv_dtype", svl.Q8_0, svl.ERR_CONFIG),
    ("n_q", 0, svl.ERR_CONFIG),
    ("ff_hidden", 0, svl.ERR_CONFIG),
    # valid for the reference, outside the kernels: the caller falls back to the reference
    ("head_dim", 96, svl.UNSUPPORTED),
    ("ff_hidden", 100, svl.UNSUPPORTED),
    ("d_model", 8192, svl.UNSUPPORTED),
    ("context", 20000, svl.UNSUPPORTED),
    ("n_q", 65, svl.UNSUPPORTED),
])
def test_config_errors_before_device_access(field, value, code):
    """Errors and the positive "unsupported" status (SVL/nn/kernels/matvec.rs:12-17 returns None to
    fall back) are decided on the host before any device call."""
    cfg = W.S1_SMALL.config(0)
    cfg[field] = value
    with pytest.raises(svl.SvlError) as e:
        svl.Model(cfg, {}, kv_dtype=cfg.get("kv_dtype", 0))
    assert e.value.code == code
    assert isinstance(e.value, svl.SvlUnsupported) == (code == svl.UNSUPPORTED)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(svl.SvlError):
        saved = svl._lib
        svl._lib = None
        try:
            svl.load_library(str(tmp_path / "libsvl.so"))
        finally:
            svl._lib = saved
