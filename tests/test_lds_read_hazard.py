"""No LDS-read result is touched before the wait that covers it, in the built library.

The fp16 GEMM main loop (nimbleml_amd/csrc/gemm_big.hpp) reads its MFMA fragments with
``asm volatile("ds_read_b128 ...")`` statements and waits for them with separate
``s_waitcnt lgkmcnt(N)`` statements, so that the next k step's reads overlap the current
MFMAs. The compiler takes an asm output as ready as soon as the statement issues: if it
ever copied, spilled or overwrote a fragment register between the read and its wait (for
example under register pressure), the copy would read the register before the LDS data
lands — wrong results with no error. This test disassembles the gfx950 code objects of
``nimbleml_amd/_lib/libnimbleml_hip.so`` (this repository's own build) and checks, for
every ``ds_read*`` of every kernel, along every control-flow path from it (loop back
edges included), that no instruction reads or writes its destination registers before an
``s_waitcnt lgkmcnt(c)`` with ``c`` no larger than the number of LDS instructions issued
after it (LDS operations complete in issue order, so that wait guarantees this one has
landed). Compiler-generated LDS reads are checked the same way; they pass by construction.

A planted mistake (a register copy between the read and its wait) is checked to fail,
and the correct form to pass, on hand-written ISA text (CPU only)."""
import os
import re
import shutil
import struct
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "nimbleml_amd", "_lib", "libnimbleml_hip.so")
LLVM = "/opt/rocm/llvm/bin"

_INS = re.compile(r"^\s+([a-z_0-9]+)\b(.*?)\s*//\s*([0-9A-Fa-f]+):")
_FUNC = re.compile(r"^[0-9a-fA-F]+ <(.+)>:$")
_VRANGE = re.compile(r"\bv\[(\d+):(\d+)\]")
_VONE = re.compile(r"\bv(\d+)\b")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")
_MAX_LGKM = 15


def _vregs(operands):
    """VGPR indices named in an operand string (ranges and single registers)."""
    out = set()
    for a, b in _VRANGE.findall(operands):
        out.update(range(int(a), int(b) + 1))
    for a in _VONE.findall(_VRANGE.sub(" ", operands)):
        out.add(int(a))
    return out


def parse_functions(text):
    """{function: [(address, mnemonic, operands)]} from llvm-objdump -d output."""
    funcs, cur = {}, None
    for line in text.splitlines():
        m = _FUNC.match(line)
        if m:
            cur = funcs.setdefault(m.group(1), [])
            continue
        m = _INS.match(line)
        if m and cur is not None:
            cur.append((int(m.group(3), 16), m.group(1), m.group(2)))
    return funcs


def _branch_target(addr, operands):
    imm = int(operands.split()[0])
    imm = imm - 65536 if imm >= 32768 else imm
    return addr + 4 + 4 * imm


def hazards(instrs):
    """Violations in one function: (address of the ds_read, address of the offending use)."""
    index = {a: i for i, (a, _, _) in enumerate(instrs)}
    found = []
    for i, (addr, op, opnds) in enumerate(instrs):
        if not op.startswith("ds_read"):
            continue
        dst = _vregs(opnds.split(",")[0])
        if not dst:
            continue
        # walk every path: state (instruction index, LDS ops issued since the read)
        stack, seen = [(i + 1, 0)], set()
        while stack:
            j, n = stack.pop()
            while j < len(instrs):
                if (j, n) in seen:
                    break
                seen.add((j, n))
                a, o, ops = instrs[j]
                if o == "s_waitcnt":
                    m = _LGKM.search(ops)
                    if m and int(m.group(1)) <= n:
                        break  # this read has landed on this path
                    j += 1
                    continue
                if _vregs(ops) & dst:
                    found.append((addr, a))
                    break
                if o.startswith("ds_"):
                    n = min(n + 1, _MAX_LGKM + 1)
                if o == "s_endpgm" or o.startswith("s_setpc") or o.startswith("s_swappc"):
                    break
                if o == "s_branch" or o.startswith("s_cbranch"):
                    t = index.get(_branch_target(a, ops))
                    if t is None:
                        found.append((addr, a))  # a branch out of the function: unknown
                        break
                    if o == "s_branch":
                        j = t
                        continue
                    stack.append((t, n))
                j += 1
    return found


def _code_objects(lib):
    """The gfx950 code objects of the library's offload bundles (.hip_fatbin)."""
    import tempfile

    with tempfile.TemporaryDirectory() as td:
        fb = os.path.join(td, "fatbin")
        subprocess.run([os.path.join(LLVM, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fb}",
                        lib, os.path.join(td, "copy")], check=True, capture_output=True)
        data = open(fb, "rb").read()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    out = []
    p = data.find(magic)
    while p >= 0:
        n = struct.unpack_from("<Q", data, p + len(magic))[0]
        off = p + len(magic) + 8
        for _ in range(n):
            o, size, tlen = struct.unpack_from("<QQQ", data, off)
            off += 24
            triple = data[off:off + tlen].decode()
            off += tlen
            if "amdgcn" in triple and size:
                out.append((triple, data[p + o:p + o + size]))
        p = data.find(magic, p + 1)
    return out


def test_checker_catches_a_planted_copy_and_passes_the_covered_form():
    good = """
0000000000001000 <k>:
	ds_read_b128 v[10:13], v2                                  // 000000001000: D9FE0000 0A000002
	ds_read_b128 v[14:17], v2 offset:16                        // 000000001008: D9FE0010 0E000002
	v_mfma_f32_32x32x16_f16 a[0:15], v[20:23], v[24:27], a[0:15] // 000000001010: D3B70000 04023114
	s_waitcnt lgkmcnt(1)                                       // 000000001018: BF8CC17F
	v_mfma_f32_32x32x16_f16 a[0:15], v[10:13], v[24:27], a[0:15] // 00000000101C: D3B70000 0402310A
	s_waitcnt lgkmcnt(0)                                       // 000000001024: BF8CC07F
	v_mov_b32_e32 v30, v14                                     // 000000001028: 7E3C030E
	s_endpgm                                                   // 00000000102C: BF810000
"""
    assert hazards(parse_functions(good)["k"]) == []
    # the compiler copies a fragment between the read and the wait covering it
    bad = good.replace("	v_mfma_f32_32x32x16_f16 a[0:15], v[20:23]",
                       "	v_mov_b32_e32 v40, v11                                     // 00000000100C: 7E50030B\n"
                       "	v_mfma_f32_32x32x16_f16 a[0:15], v[20:23]")
    assert hazards(parse_functions(bad)["k"]) == [(0x1000, 0x100C)]
    # lgkmcnt(1) does not cover the second of two outstanding reads
    late = good.replace("v_mfma_f32_32x32x16_f16 a[0:15], v[10:13], v[24:27], a[0:15] // 00000000101C",
                        "v_mfma_f32_32x32x16_f16 a[0:15], v[14:17], v[24:27], a[0:15] // 00000000101C")
    assert hazards(parse_functions(late)["k"]) == [(0x1008, 0x101C)]
    # a loop back edge: the read at the bottom is used at the top of the next iteration
    loop = """
0000000000002000 <l>:
	s_waitcnt lgkmcnt(0)                                       // 000000002000: BF8CC07F
	v_mov_b32_e32 v1, v10                                      // 000000002004: 7E02030A
	ds_read_b32 v10, v2                                        // 000000002008: D86C0000 0A000002
	s_cbranch_scc1 65531                                       // 000000002010: BF85FFFB
	s_endpgm                                                   // 000000002014: BF810000
"""
    assert hazards(parse_functions(loop)["l"]) == []
    unguarded = loop.replace("	s_waitcnt lgkmcnt(0)                                       // 000000002000: BF8CC07F\n", "")
    unguarded = unguarded.replace("65531", "65532")  # the back edge lands on the copy
    assert hazards(parse_functions(unguarded)["l"]) == [(0x2008, 0x2004)]


def test_no_lds_read_result_is_used_before_its_wait():
    objdump = os.path.join(LLVM, "llvm-objdump")
    if not (os.path.exists(objdump) and shutil.which("true")):
        pytest.skip("llvm-objdump not available")
    if not os.path.exists(LIB):
        pytest.skip("library not built (python nimbleml_amd/build.py)")
    import tempfile

    objs = _code_objects(LIB)
    assert objs, "no device code objects in the library"
    checked, bad = 0, []
    with tempfile.TemporaryDirectory() as td:
        for k, (triple, blob) in enumerate(objs):
            assert triple.endswith("gfx950"), triple
            path = os.path.join(td, f"co{k}.elf")
            open(path, "wb").write(blob)
            text = subprocess.run([objdump, "-d", "--mcpu=gfx950", path], check=True,
                                  capture_output=True, text=True).stdout
            for name, instrs in parse_functions(text).items():
                checked += sum(1 for _, o, _ in instrs if o.startswith("ds_read"))
                bad += [(name, hex(r), hex(u)) for r, u in hazards(instrs)]
    print(f"{checked} LDS reads checked")
    assert checked > 1000
    assert not bad, bad[:20]
