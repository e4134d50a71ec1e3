"""The C ABI: libckl_hip.so loads without a GPU, exports every function include/ckl_hip.h
declares, the Python binding declares each one, and the host-entry call sequence packs
constants byte-exactly (tests/MLIR/test_exec_to_llvm.py:57-65 of the reference)."""
import ctypes
import re
from pathlib import Path

import pytest

import ckl
from ckl import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "ckl_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ckl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _native.native()
    names = declared_functions()
    assert len(names) >= 40
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.EXPORTED, f"{name} is not bound in ckl/_native.py"
    assert lib.ckl_abi_version() == 1


def test_kernel_library_is_present():
    assert _native.library_identity().startswith("ckl.hip.library.")


def test_missing_kernel_library_fails_loudly(tmp_path):
    """Library-selected kernels never fall back silently when the gfx950 code object is absent."""
    import os
    import subprocess
    import sys
    root = Path(__file__).resolve().parents[1]
    code = ("import sys; sys.path[:0] = ['composable-kernel-language_amd/python', 'composable-kernel-language_amd']\n"
            "from programs import vector_pipeline as vp\n"
            "try:\n    vp.lower(1024).compile(fuse_pointwise=False)\nexcept RuntimeError as e:\n"
            "    print('raised', e)\n")
    env = dict(os.environ, CKL_KERNEL_LIBRARY=str(tmp_path / "absent.hsaco"))
    out = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True, text=True, timeout=120)
    assert "raised" in out.stdout and "kernel library" in out.stdout, out.stdout + out.stderr


def test_errors_map_to_python_exceptions():
    with pytest.raises(RuntimeError, match="unknown pass"):
        _native.native_opt("module {\n}\n", ["no-such-pass"])
    out = ctypes.c_void_p()
    status = _native.native().ckl_compile(b"module {\n}\n", None, ctypes.byref(out))
    assert status == 3 and b"at least one marked CKL kernel" in _native.native().ckl_last_error()


I64 = ckl.Buffer[ckl.i64, (4,)]
F64 = ckl.Buffer[ckl.f64, (4,)]


@ckl.kernel
def mixed(dst: I64, values: F64, offset: ckl.i64, scale: ckl.f64) -> None:
    i = ckl.global_id(0)
    if i < 4:
        dst[i] = dst[i] + offset
        values[i] = values[i] * scale


@ckl.program
def constants(dst: I64, values: F64) -> None:
    ckl.launch(mixed, dst, values, -7, -0.0, grid=(1,), block=(4,))


def test_host_entry_packs_constants_little_endian():
    compiled = constants.lower(signature={"dst": ckl.BufferSpec((4,), ckl.i64),
                                          "values": ckl.BufferSpec((4,), ckl.f64)}).compile()
    host = compiled.host_ir.splitlines()
    calls = [line.split("(")[0] for line in host]
    assert calls == ["ckl_module", "ckl_resource", "ckl_resource", "ckl_kernel", "ckl_argument_resource",
                     "ckl_argument_resource", "ckl_argument_value", "ckl_argument_value", "ckl_commit"]
    assert "ckl_argument_value([F9 FF FF FF FF FF FF FF], 8)" in host
    assert "ckl_argument_value([00 00 00 00 00 00 00 80], 8)" in host
    assert "extern \"C\" __global__" in compiled.device_ir
