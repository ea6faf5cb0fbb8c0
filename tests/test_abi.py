"""C-ABI checks that run without a GPU: the library loads, exports every
entry point include/ane_hip.h declares, and its host-side layout functions
agree with the Python mirror and the oracle.  No device call is made."""
import ctypes
import os
import re

import numpy as np

import ane
from ane import _lib
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    inc = os.path.join(ROOT, "include")
    for fn in sorted(os.listdir(inc)):
        if not fn.endswith(".h"):
            continue
        src = open(os.path.join(inc, fn)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(ane_\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("ane_open", "ane_close", "ane_eval_logits", "ane_eval_loss", "ane_set_params"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers each of them
    assert sorted(_lib.SIGNATURES) == declared_functions()
    _lib.load()


def test_param_layout_matches_python_and_oracle():
    lib = _lib.load()
    for arch in ("llama2", "nanochat"):
        for cfg in (ane.tiny(arch), ane.stories110m(arch), ane.tiny(arch, layers=3)):
            mc = _lib.model_cfg(cfg)
            n = lib.ane_param_count(ctypes.byref(mc))
            assert n == ane.param_count(cfg) == oracle.param_count(cfg)
            nseg = lib.ane_param_layout(ctypes.byref(mc), None, None, 0)
            off = (ctypes.c_int64 * nseg)()
            sz = (ctypes.c_int64 * nseg)()
            lib.ane_param_layout(ctypes.byref(mc), off, sz, nseg)
            got = [(off[i], sz[i]) for i in range(nseg)]
            assert got == oracle.param_segments(cfg)
            assert got == [(o, int(np.prod(s))) for _, o, s in ane.param_layout(cfg)]


def test_open_requires_weights():
    try:
        ane.Open(ane.Options())
    except ane.EngineError as e:
        assert str(e) == "storiesane open: model path is empty"
    else:
        raise AssertionError("Open without weights must fail")


def test_code_object_arg_structs_match_the_kernels():
    """The ctypes mirrors of include/ane_kernels.h's argument structs (what a
    host that launches the code objects itself passes) against the layout
    the kernels were compiled with."""
    from ane import hsaco
    hsaco.check_abi()


def test_code_objects_hold_the_kernel_table():
    """Every kernel include/ane_kernels.h names is a global kernel of one of
    the built code objects (gfx950 ELF)."""
    from ane import hsaco
    src = open(os.path.join(ROOT, "include", "ane_kernels.h")).read()
    names = sorted(n for n in set(re.findall(r"\b(ane_k_\w+)", src)) if not n.endswith("_"))
    assert len(names) >= 9
    blobs = []
    for fname in hsaco.MODULES.values():
        data = open(os.path.join(hsaco.HERE, fname), "rb").read()
        assert data[:4] == b"\x7fELF", fname
        blobs.append(data)
    for n in names:
        assert any((n + ".kd").encode() in b for b in blobs), n
