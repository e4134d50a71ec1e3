"""The executor's reader of kernel argument layouts (csrc/runtime/kernarg.cpp), which every launch
is checked against, agrees with LLVM's own dump of the same code object's metadata note, for
every kernel of the gfx950 library, also inside an offload bundle; malformed images are refused.
No GPU needed."""
import ctypes
import shutil
import struct
import subprocess
from pathlib import Path

import pytest
import yaml

from ckl import _native

HSACO = Path(_native.__file__).resolve().parent / "_lib" / "ckl_kernels_gfx950.hsaco"
READELF = shutil.which("llvm-readelf") or "/opt/rocm/llvm/bin/llvm-readelf"


def layout(image: bytes, kernel: str):
    lib = _native.native()
    offsets, sizes = (ctypes.c_uint32 * 64)(), (ctypes.c_uint32 * 64)()
    count, segment = ctypes.c_uint64(), ctypes.c_uint32()
    buffer = ctypes.create_string_buffer(image, len(image))
    _native.check(lib.ckl_code_object_arguments(buffer, len(image), kernel.encode(), offsets, sizes, 64,
                                                ctypes.byref(count), ctypes.byref(segment)))
    return [(offsets[k], sizes[k]) for k in range(count.value)], segment.value


def llvm_metadata(path: Path) -> dict:
    text = subprocess.run([READELF, "--notes", str(path)], capture_output=True, text=True, check=True).stdout
    document = text[text.index("---"):]
    document = document[:document.index("\n...")] if "\n..." in document else document
    kernels = yaml.safe_load(document)["amdhsa.kernels"]
    return {k[".name"]: ([(a[".offset"], a[".size"]) for a in k.get(".args", [])
                          if not a[".value_kind"].startswith("hidden_")], k[".kernarg_segment_size"]) for k in kernels}


@pytest.fixture(scope="module")
def library():
    if not HSACO.exists():
        pytest.skip("kernel library not built")
    if not Path(READELF).exists():
        pytest.skip("llvm-readelf not available")
    return HSACO.read_bytes(), llvm_metadata(HSACO)


def test_reader_matches_llvm_for_every_library_kernel(library):
    image, expected = library
    assert len(expected) > 50
    for name, (args, segment) in expected.items():
        assert layout(image, name) == (args, segment), name
        # Library convention: one by-value argument block, a multiple of 8 bytes (aligned(8) structs).
        assert len(args) == 1 and args[0][0] == 0 and args[0][1] % 8 == 0, name


def test_reader_finds_the_gfx950_entry_of_an_offload_bundle(library):
    image, expected = library
    host = b"\x7fELF-host-placeholder"
    ids = [b"host-x86_64-unknown-linux-gnu-", b"hipv4-amdgcn-amd-amdhsa--gfx950"]
    header_size = 24 + 8 + sum(24 + len(i) for i in ids)
    entries, payload, offset = b"", b"", header_size
    for ident, blob in zip(ids, (host, image)):
        entries += struct.pack("<QQQ", offset, len(blob), len(ident)) + ident
        payload += blob
        offset += len(blob)
    bundle = b"__CLANG_OFFLOAD_BUNDLE__" + struct.pack("<Q", len(ids)) + entries + payload
    name = sorted(expected)[0]
    assert layout(bundle, name) == expected[name]


@pytest.mark.parametrize("image", [b"not an elf at all", b"\x7fELF" + b"\0" * 60,
                                   b"__CLANG_OFFLOAD_BUNDLE__" + struct.pack("<Q", 1) + struct.pack("<QQQ", 0, 10**9, 3) + b"abc"])
def test_malformed_images_are_refused(image):
    with pytest.raises(ValueError, match="code object"):
        layout(image, "anything")


def test_unknown_kernel_is_refused(library):
    image, _ = library
    with pytest.raises(ValueError, match="no kernel"):
        layout(image, "ckl_no_such_kernel")


def test_truncated_metadata_is_refused(library):
    image, _ = library
    with pytest.raises(ValueError):
        layout(image[: len(image) // 3], "ckl_embedding")
