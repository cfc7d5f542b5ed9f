"""Build check: every kernel the host side of libmace_hip.so registers with the HIP
runtime exists in the library's gfx950 code objects.

The runtime looks kernels up by mangled name at their first launch and aborts the
process when one is missing -- which happens when host and device compilation
mangle a kernel's name differently (for instance a kernel parameter type that
depends on an unnamed enum).  The check reads the ELF sections of the library
directly: host names from its read-only string sections, device names from the
symbol tables of the code objects in the offload bundles of .hip_fatbin.

    python3 check_kernel_symbols.py [path/to/libmace_hip.so]
"""

from __future__ import annotations

import re
import struct
import sys
from pathlib import Path

BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
KERNEL_RE = re.compile(rb"_ZN4mace(?:12_GLOBAL__N_1)?\d+k_[0-9A-Za-z_$.]+")


def elf_sections(data: bytes) -> dict:
    """{name: bytes} of an ELF64 little-endian image."""
    if data[:4] != b"\x7fELF" or data[4] != 2 or data[5] != 1:
        raise ValueError("not an ELF64 little-endian file")
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", data, 0x3A)
    hdrs = []
    for i in range(shnum):
        name, typ, flags, addr, off, size, link, info, align, entsize = struct.unpack_from(
            "<IIQQQQIIQQ", data, shoff + i * shentsize)
        hdrs.append((name, typ, off, size, link))
    strtab = hdrs[shstrndx]
    names = data[strtab[2]:strtab[2] + strtab[3]]
    out = {}
    for name, typ, off, size, link in hdrs:
        nm = names[name:names.index(b"\0", name)].decode()
        out[nm] = (typ, data[off:off + size] if typ != 8 else b"", link)  # 8 = SHT_NOBITS
    return out


def func_symbols(code_object: bytes) -> set:
    secs = elf_sections(code_object)
    syms = secs[".symtab"][1]
    strs = secs[".strtab"][1]
    out = set()
    for k in range(0, len(syms), 24):
        st_name, st_info = struct.unpack_from("<IB", syms, k)
        if st_info & 0xF == 2:  # STT_FUNC
            out.add(strs[st_name:strs.index(b"\0", st_name)].decode())
    return out


def device_kernels(lib: bytes, target: str = "gfx950") -> set:
    fatbin = elf_sections(lib)[".hip_fatbin"][1]
    out = set()
    pos = fatbin.find(BUNDLE_MAGIC)
    while pos >= 0:
        n, = struct.unpack_from("<Q", fatbin, pos + 24)
        p = pos + 32
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            triple = fatbin[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if triple.endswith(target):
                out |= func_symbols(fatbin[pos + off:pos + off + size])
        pos = fatbin.find(BUNDLE_MAGIC, pos + 1)
    return out


def host_kernels(lib: bytes) -> set:
    out = set()
    for name, (typ, body, _) in elf_sections(lib).items():
        if name.startswith(".rodata"):
            out |= {m.decode() for m in KERNEL_RE.findall(body)}
    return out


def check(path) -> list:
    data = Path(path).read_bytes()
    host, dev = host_kernels(data), device_kernels(data)
    if not host or not dev:
        raise RuntimeError(f"{path}: found {len(host)} host and {len(dev)} device kernel names")
    return sorted(host - dev)


if __name__ == "__main__":
    lib = sys.argv[1] if len(sys.argv) > 1 else str(Path(__file__).resolve().parents[1] /
                                                     "mace_mlx_amd" / "_lib" / "libmace_hip.so")
    missing = check(lib)
    for m in missing:
        print("kernel registered by the host but absent from the gfx950 code object:", m)
    sys.exit(1 if missing else 0)
