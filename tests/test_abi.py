"""The C ABI library without a GPU: it loads, exports every entry point the header
declares, and rejects unsupported or invalid requests with the documented codes
before touching the device."""
import ctypes
import os
import re

import pytest

from mi_qmm import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def header_symbols():
    text = "".join(open(os.path.join(INCLUDE, h)).read()
                   for h in sorted(os.listdir(INCLUDE)) if h.endswith(".h"))
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|void|const char\*)\s+(mi_\w+)\s*\(",
                                 text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(L.LIB_PATH):
        pytest.fail(f"{L.LIB_PATH} not built (run __graft_entry__.build())")
    return L.lib()


def test_exports_every_header_symbol(lib):
    syms = header_symbols()
    assert len(syms) >= 10 and "mi_ckpt_open" in syms and "mi_ckpt_close" in syms
    for s in syms:
        assert hasattr(lib, s), s


def test_version_and_empty_error(lib):
    assert lib.mi_version().decode()


def _qmm(lib, **kw):
    a = dict(y=1, x=1, w=1, s=1, b=1, M=1, N=64, K=256, transpose=True, gs=L.opt(64),
             bits=L.opt(4), mode=b"affine", xd=L.DT_BFLOAT16, sbd=L.DT_BFLOAT16)
    a.update(kw)
    P = ctypes.c_void_p
    return lib.mi_quantized_matmul(P(a["y"]), P(a["x"]), P(a["w"]), P(a["s"]), P(a["b"]),
                                   a["M"], a["N"], a["K"], a["transpose"], a["gs"], a["bits"],
                                   a["mode"], a["xd"], a["sbd"], None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(mode=b"nf4"), L.MI_ERR_UNSUPPORTED, "mode"),
    (dict(mode=b"mxfp4", gs=L.opt(32)), L.MI_ERR_UNSUPPORTED, "uint8"),
    (dict(mode=b"mxfp4", gs=L.opt(64)), L.MI_ERR_INVALID, "group_size=32"),
    (dict(transpose=False), L.MI_ERR_UNSUPPORTED, "transpose"),
    (dict(bits=L.opt(7)), L.MI_ERR_UNSUPPORTED, "bits"),
    (dict(bits=L.opt(3), xd=L.DT_FLOAT32), L.MI_ERR_UNSUPPORTED, "bf16 activations"),
    (dict(gs=L.opt(16)), L.MI_ERR_UNSUPPORTED, "group_size"),
    (dict(K=100), L.MI_ERR_INVALID, "multiple"),
    (dict(xd=L.DT_FLOAT16), L.MI_ERR_UNSUPPORTED, "dtype"),
    (dict(sbd=L.DT_FLOAT32), L.MI_ERR_UNSUPPORTED, "dtype"),
    (dict(M=-1), L.MI_ERR_INVALID, "negative"),
    (dict(y=0), L.MI_ERR_INVALID, "null"),
])
def test_qmm_rejections(lib, kw, code, msg):
    assert _qmm(lib, **kw) == code
    assert msg in lib.mi_last_error().decode()


def test_qmm_defaults_and_empty_calls_are_noops(lib):
    # mlx_optional_int without a value means group_size 64 / bits 4; empty shapes return 0
    assert _qmm(lib, M=0, gs=L.opt(None), bits=L.opt(None)) == L.MI_OK
    assert _qmm(lib, N=0) == L.MI_OK


def test_gather_rejections(lib):
    P = ctypes.c_void_p
    args = [P(1)] * 5 + [None, None]
    rc = lib.mi_gather_qmm(*args, 4, 0, 1, 1, 64, 256, 2, True, L.opt(64), L.opt(4), b"affine",
                           True, L.DT_BFLOAT16, L.DT_BFLOAT16, None)
    assert rc == L.MI_ERR_INVALID and "lhs_div" in lib.mi_last_error().decode()
    rc = lib.mi_gather_qmm(*args, 0, 1, 1, 1, 64, 256, 2, True, L.opt(64), L.opt(4), b"affine",
                           True, L.DT_BFLOAT16, L.DT_BFLOAT16, None)
    assert rc == L.MI_OK


def test_geometry_solve_matches_oracle(lib):
    import oracle as O
    b, g = ctypes.c_int(0), ctypes.c_int(0)
    for w_cols, s_cols, in_dim in [(512, 64, 4096), (1024, 64, 4096), (320, 16, 2048),
                                   (384, 16, 2048), (256, 32, 2048), (320, 16, 3000),
                                   (100, 7, 4096), (448, 56, 7168), (0, 1, 1)]:
        rc = lib.mi_affine_params_from_geometry(w_cols, s_cols, in_dim, ctypes.byref(b),
                                                ctypes.byref(g))
        want = O.affine_params_from_geometry(w_cols, s_cols, in_dim)
        if want is None:
            assert rc == L.MI_ERR_INVALID
        else:
            assert rc == L.MI_OK and (b.value, g.value) == want


def test_python_wrapper_fails_loudly_without_library(tmp_path, monkeypatch):
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(ImportError):
        L.lib()
