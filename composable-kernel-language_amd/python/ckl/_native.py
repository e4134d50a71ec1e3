"""ctypes binding of the C ABI in include/ckl_hip.h (libckl_hip.so).

The reference binds its native layer through nanobind (lib/Compiler/RuntimeBindings.cpp:56-105);
this module declares the same surface as plain C functions. The library is loaded from
python/ckl/_lib/ (built in-tree by build.py) or from CKL_NATIVE_LIBRARY. There is no
Python fallback: every entry point fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_library = None

LIB_DIR = Path(__file__).resolve().parent / "_lib"
LIBRARY_NAME = "libckl_hip.so"


class CompileOptions(ctypes.Structure):
    _fields_ = [("reuse_storage", ctypes.c_int), ("fuse_pointwise", ctypes.c_int), ("strict", ctypes.c_int),
                ("chip", ctypes.c_char_p)]


class Argument(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("buffer", ctypes.c_void_p), ("integer", ctypes.c_int64), ("real", ctypes.c_double)]


class StorageResource(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_uint64), ("alignment", ctypes.c_uint64), ("device", ctypes.c_int), ("kind", ctypes.c_int),
                ("address_space", ctypes.c_char_p), ("users", ctypes.POINTER(ctypes.c_uint64)), ("user_count", ctypes.c_size_t)]


class StorageAssignment(ctypes.Structure):
    _fields_ = [("heap", ctypes.c_uint64), ("offset", ctypes.c_uint64), ("slot", ctypes.c_uint64),
                ("shares_first", ctypes.c_uint64)]


ENTRY = ctypes.CFUNCTYPE(None, ctypes.POINTER(ctypes.c_void_p))

_SIGNATURES = {
    "ckl_abi_version": ([], ctypes.c_int),
    "ckl_last_error": ([], ctypes.c_char_p),
    "ckl_string_free": ([ctypes.c_void_p], None),
    "ckl_compile": ([ctypes.c_char_p, ctypes.POINTER(CompileOptions), ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_program_ir": ([ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_size_t)],
                       ctypes.c_int),
    "ckl_program_signature": ([ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.POINTER(ctypes.c_uint64)),
                               ctypes.POINTER(ctypes.POINTER(ctypes.c_char_p))], ctypes.c_int),
    "ckl_program_from_entry": ([ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_char_p),
                                ctypes.c_size_t, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_program_release": ([ctypes.c_void_p], None),
    "ckl_opt": ([ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_plan_storage": ([ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t, ctypes.POINTER(StorageResource),
                          ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                          ctypes.POINTER(StorageAssignment)], ctypes.c_int),
    "ckl_library_identity": ([], ctypes.c_char_p),
    "ckl_device_count": ([], ctypes.c_int),
    "ckl_device_open": ([ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_device_name": ([ctypes.c_void_p], ctypes.c_char_p),
    "ckl_device_release": ([ctypes.c_void_p], None),
    "ckl_buffer_alloc": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_buffer_import": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_buffer_slice": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_buffer_address": ([ctypes.c_void_p], ctypes.c_uint64),
    "ckl_buffer_nbytes": ([ctypes.c_void_p], ctypes.c_uint64),
    "ckl_buffer_copy_from_host": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64], ctypes.c_int),
    "ckl_buffer_copy_to_host": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64], ctypes.c_int),
    "ckl_buffer_release": ([ctypes.c_void_p], None),
    "ckl_bind": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(Argument), ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)],
                 ctypes.c_int),
    "ckl_bind_static": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(Argument), ctypes.c_size_t, ctypes.c_void_p,
                         ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "ckl_static_scratch_bytes": ([], ctypes.c_uint64),
    "ckl_invocation_run": ([ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64], ctypes.c_int),
    "ckl_invocation_benchmark": ([ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64,
                                  ctypes.POINTER(ctypes.c_double)], ctypes.c_int),
    "ckl_invocation_node_count": ([ctypes.c_void_p], ctypes.c_uint64),
    "ckl_profiler_region": ([ctypes.c_int], ctypes.c_int),
    "ckl_invocation_rebind": ([ctypes.c_void_p, ctypes.POINTER(Argument), ctypes.c_size_t], ctypes.c_int),
    "ckl_invocation_graph_instantiations": ([ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "ckl_invocation_memory": ([ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "ckl_invocations_run": ([ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64,
                             ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_double)], ctypes.c_int),
    "ckl_invocation_launch_count": ([ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
                                    ctypes.c_int),
    "ckl_invocation_edge_count": ([ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
                                  ctypes.c_int),
    "ckl_code_object_arguments": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32),
                                   ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64),
                                   ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int),
    "ckl_invocation_time_node": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)],
                                 ctypes.c_int),
    "ckl_invocation_node_name": ([ctypes.c_void_p, ctypes.c_uint64], ctypes.c_char_p),
    "ckl_invocation_unit_count": ([ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "ckl_invocation_unit_name": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_char_p)], ctypes.c_int),
    "ckl_invocation_unit_members": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64), ctypes.c_uint64,
                                     ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "ckl_invocation_time_unit": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)],
                                 ctypes.c_int),
    "ckl_invocation_profile_units": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double), ctypes.c_uint64,
                                      ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "ckl_invocation_release": ([ctypes.c_void_p], None),
    "ckl_begin": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64], None),
    "ckl_module": ([ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_uint64], None),
    "ckl_heap": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64], None),
    "ckl_resource": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p], None),
    "ckl_kernel": ([ctypes.c_void_p, ctypes.c_char_p] + [ctypes.c_uint64] * 7, None),
    "ckl_argument_resource": ([ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64], None),
    "ckl_argument_value": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64], None),
    "ckl_dependency": ([ctypes.c_void_p, ctypes.c_uint64], None),
    "ckl_commit": ([ctypes.c_void_p, ctypes.c_uint64], None),
    "ckl_workspace": ([ctypes.c_void_p, ctypes.c_uint64], None),
}
EXPORTED = tuple(_SIGNATURES)


def library_path() -> Path:
    configured = os.environ.get("CKL_NATIVE_LIBRARY")
    return Path(configured) if configured else LIB_DIR / LIBRARY_NAME


def native():
    """Load libckl_hip.so (once). Raises RuntimeError when it has not been built."""
    global _library
    if _library is not None:
        return _library
    path = library_path()
    if not path.is_file():
        raise RuntimeError(f"CKL native library is not built ({path}); run composable-kernel-language_amd/build.py "
                           "or __graft_entry__.build()")
    library = ctypes.CDLL(str(path))
    for name, (argtypes, restype) in _SIGNATURES.items():
        function = getattr(library, name)
        function.argtypes = argtypes
        function.restype = restype
    if library.ckl_abi_version() != 1:
        raise RuntimeError("CKL native library ABI version mismatch")
    _library = library
    return library


class NativeError(RuntimeError):
    pass


def check(status: int) -> None:
    if status == 0:
        return
    message = native().ckl_last_error().decode(errors="replace")
    if status == 1:
        raise ValueError(message)
    raise NativeError(message)


def native_opt(ir: str, passes) -> str:
    lib = native()
    out = ctypes.c_void_p()
    check(lib.ckl_opt(ir.encode(), ";".join(passes).encode(), ctypes.byref(out)))
    try:
        return ctypes.string_at(out.value).decode()
    finally:
        lib.ckl_string_free(out)


NONE = (1 << 64) - 1


def plan_storage(node_count, edges, resources, reuse=True):
    """Run the native storage planner. `resources`: dicts with bytes, alignment, kind
    ("temporary" | "persistent" | "external"), users, optional device and address_space.
    Returns (baseline_bytes, planned_bytes, [assignment dict or None per resource])."""
    kinds = {"temporary": 0, "persistent": 1, "external": 2}
    flat = (ctypes.c_uint64 * max(1, 2 * len(edges)))(*[v for e in edges for v in e])
    keep = []
    table = (StorageResource * max(1, len(resources)))()
    for k, r in enumerate(resources):
        users = (ctypes.c_uint64 * max(1, len(r["users"])))(*r["users"])
        keep.append(users)
        table[k] = StorageResource(r["bytes"], r.get("alignment", 256), r.get("device", 0), kinds[r.get("kind", "temporary")],
                                   r.get("address_space", "global").encode(), users, len(r["users"]))
    out = (StorageAssignment * max(1, len(resources)))()
    baseline, planned = ctypes.c_uint64(), ctypes.c_uint64()
    check(native().ckl_plan_storage(node_count, flat, len(edges), table, len(resources), int(reuse),
                                    ctypes.byref(baseline), ctypes.byref(planned), out))
    result = []
    for k in range(len(resources)):
        a = out[k]
        result.append(None if a.heap == NONE else dict(heap=a.heap, offset=a.offset, slot=a.slot,
                                                       shares_first=None if a.shares_first == NONE else a.shares_first))
    return baseline.value, planned.value, result


def library_identity() -> str:
    return native().ckl_library_identity().decode()


def device_count() -> int:
    return int(native().ckl_device_count())
