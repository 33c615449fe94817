"""No 12- or 16-byte vector-memory store in the built library is directly followed by an instruction that writes one
of its data registers (CPU only: the device code objects of voxrt_amd/libvoxrt_hip.so are disassembled with the
ROCm LLVM tools).

A VMEM store of more than 8 bytes may read its data registers after it issues; a VALU write of one of them right
behind the store can then reach memory in place of the stored value. It showed as nondeterministic wrong outputs in
the fourth dword of the streaming GEMM's SiLU stores with two workgroups per CU. The kernels store through
store_b128_sep / store16_sep (vx_internal.h), which pin two wait states after the store; this test checks that the
compiled code holds no instance of the pattern anywhere."""
import os
import re
import shutil
import struct
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SO = os.path.join(ROOT, "voxrt_amd", "libvoxrt_hip.so")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

_STORE = re.compile(r"^\s+(?:buffer|global|flat|scratch)_store_dwordx[34]\s+(?:v\[\d+:\d+\],\s*)?v\[(\d+):(\d+)\]")
_WRITE = re.compile(r"^\s+(?:v_\w+|ds_read\w*|buffer_load\w*|global_load\w*|flat_load\w*|scratch_load\w*)"
                    r"\s+v(?:\[(\d+):(\d+)\]|(\d+)\b)")


def store_hazards(lines):
    """(function, store, next instruction) for each wide store whose next instruction writes its data VGPRs."""
    func, pend, hits = None, None, []
    for line in lines:
        if line[:1].isalnum() and line.rstrip().endswith(">:"):
            func, pend = line.split("<", 1)[1].split(">", 1)[0], None
            continue
        if not line.startswith(("\t", " ")) or not line.strip() or line.strip().startswith(";"):
            continue
        if pend is not None:
            w = _WRITE.match(line)
            if w:
                lo, hi = (int(w.group(3)),) * 2 if w.group(3) else (int(w.group(1)), int(w.group(2)))
                if not (hi < pend[0] or lo > pend[1]):
                    hits.append((func, pend[2], line.strip()))
            pend = None
        s = _STORE.match(line)
        if s:
            pend = (int(s.group(1)), int(s.group(2)), line.strip())
    return hits


def _code_objects(fatbin):
    """The gfx950 code objects of the clang offload bundles concatenated in a .hip_fatbin section."""
    magic, out, pos = b"__CLANG_OFFLOAD_BUNDLE__", [], 0
    while (i := fatbin.find(magic, pos)) >= 0:
        (n,) = struct.unpack_from("<Q", fatbin, i + len(magic))
        p = i + len(magic) + 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            triple = fatbin[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if triple == TARGET and size:
                out.append(fatbin[i + off:i + off + size])
        pos = i + len(magic)
    return out


def test_scanner_flags_a_store_followed_by_a_write_of_its_data():
    asm = ["0000000000001000 <k>:",
           "\tbuffer_store_dwordx4 v[4:7], v1, s[8:11], 0 offen",
           "\tv_add_f32_e32 v7, v2, v3",
           "\tglobal_store_dwordx4 v[8:9], v[0:3], off",
           "\ts_nop 1",
           "\tv_mov_b32_e32 v0, 0",
           "\tglobal_store_dwordx2 v[8:9], v[0:1], off",
           "\tv_mov_b32_e32 v0, 0",
           "\tglobal_store_dwordx3 v[8:9], v[0:2], off",
           "\tv_mfma_i32_16x16x64_i8 v[0:3], v[10:13], v[14:17], v[0:3]"]
    hits = store_hazards(asm)
    assert [h[1].split()[0] for h in hits] == ["buffer_store_dwordx4", "global_store_dwordx3"]


def test_library_has_no_wide_store_followed_by_a_write_of_its_data():
    if not os.path.exists(SO):
        pytest.skip("libvoxrt_hip.so is not built")
    if not (os.path.exists(os.path.join(LLVM, "llvm-objcopy")) and os.path.exists(os.path.join(LLVM, "llvm-objdump"))):
        pytest.skip("ROCm LLVM tools are not installed")
    tmp = tempfile.mkdtemp()
    try:
        fat = os.path.join(tmp, "fat.bin")
        subprocess.run([os.path.join(LLVM, "llvm-objcopy"), "--dump-section", f".hip_fatbin={fat}", SO,
                        os.path.join(tmp, "copy.so")], check=True, capture_output=True)
        objs = _code_objects(open(fat, "rb").read())
        assert len(objs) >= 6, "expected one gfx950 code object per device source"
        stores, hits = 0, []
        for k, co in enumerate(objs):
            path = os.path.join(tmp, f"{k}.co")
            open(path, "wb").write(co)
            text = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", path],
                                  check=True, capture_output=True, text=True).stdout.splitlines()
            stores += sum(1 for line in text if _STORE.match(line))
            hits += store_hazards(text)
        assert stores > 1000, "the streaming and small-token GEMMs store 16-byte blocks"
        assert not hits, "\n".join(f"{f}: {s} / {w}" for f, s, w in hits[:10])
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
