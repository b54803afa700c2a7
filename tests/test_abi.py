"""The C ABI library loads and exports every entry point include/vgo.h declares.

CPU only: nothing here launches a kernel.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from tests.conftest import ROOT, import_package

HEADER = ROOT / "include" / "vgo.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vgo_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "vgo_mass_bias_attn_fwd" in names and "vgo_top4_project" in names


def test_library_exports_every_declared_symbol():
    lib_mod = import_package("_lib")
    lib = lib_mod.load()
    missing = [name for name in declared_symbols() if not hasattr(lib, name)]
    assert not missing, f"libvgo.so lacks {missing}"
    # The binding declares a signature for each of them, too.
    assert set(declared_symbols()) <= set(lib_mod.SIGNATURES)


def test_abi_version_matches_header():
    lib = import_package("_lib").load()
    version = int(re.search(r"#define VGO_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.vgo_abi_version() == version


def test_argument_errors_raise_value_error_without_a_gpu():
    # Validation happens on the host before any launch, so this runs on CPU.
    lib_mod = import_package("_lib")
    lib = lib_mod.load()
    status = lib.vgo_mass_bias_attn_fwd(None, None, None, None, None, 1, 1, 1, 1, 32,
                                        (ctypes.c_int64 * 3)(), (ctypes.c_int64 * 3)(),
                                        (ctypes.c_int64 * 3)(), (ctypes.c_int64 * 3)(), 1, None)
    assert status == lib_mod.VGO_EINVAL
    assert "head_dim=64" in lib_mod.last_error()
    with pytest.raises(ValueError, match="head_dim=64"):
        lib_mod.check(status)


def test_cpu_tensors_are_rejected():
    vgo = import_package()
    import torch
    q = torch.zeros(1, 1, 4, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        vgo.mass_bias_attention(q, q, q, torch.zeros(4))


def dynamic_exports(path: Path) -> set[str]:
    """Names of the defined global/weak symbols of default or protected visibility in an
    ELF64 little-endian shared object's .dynsym (what the dynamic linker resolves)."""
    import struct
    data = path.read_bytes()
    assert data[:4] == b"\x7fELF" and data[4] == 2 and data[5] == 1, "not an ELF64 LE object"
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    sections = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    names = set()
    for sh_name, sh_type, _, _, offset, size, link, _, _, entsize in sections:
        if sh_type != 11:  # SHT_DYNSYM
            continue
        strtab = sections[link]
        str_off = strtab[4]
        for i in range(1, size // entsize):
            st_name, st_info, st_other, st_shndx, _, _ = struct.unpack_from("<IBBHQQ", data, offset + i * entsize)
            if st_shndx == 0 or (st_info >> 4) not in (1, 2) or (st_other & 3) in (1, 2):
                continue  # undefined, local, hidden or internal
            end = data.index(b"\0", str_off + st_name)
            names.add(data[str_off + st_name:end].decode())
    return names


def test_library_symbols_are_only_the_c_abi():
    """The shared object's dynamic symbol table holds the vgo_* C entry points the
    header declares and nothing else (no C++ helpers, no compiler unit ids)."""
    lib_path = Path(import_package("_lib").LIBRARY_PATH)
    exports = dynamic_exports(lib_path)
    assert set(declared_symbols()) <= exports
    extra = sorted(name for name in exports if not name.startswith("vgo_"))
    assert not extra, f"libvgo.so exports non-ABI symbols: {extra[:10]}"
    undeclared = sorted(exports - set(declared_symbols()))
    assert not undeclared, f"libvgo.so exports symbols include/vgo.h does not declare: {undeclared}"
