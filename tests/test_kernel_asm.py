"""Checks on the library's own generated gfx950 code (no GPU needed).

The projection kernel takes work tickets with a vector atomic written as an
inline asm statement (ticket_take) that the compiler's wait-counter
bookkeeping does not see, and waits for it later with an explicit
`s_waitcnt vmcnt(N)` (ticket_wait). The atomic's result register is not
ready until that wait, which the compiler does not know, so nothing between
the two may read, copy, spill or overwrite it. These tests compile
csrc/dz_kernels.hip to assembly with the library's own flags and check every
such pair:
  * a wait follows the atomic in the same function;
  * from the atomic to its first wait in layout order, no instruction names
    the ticket register except the zero-initialisation of the paths where
    no ticket is taken, and at least N vector-memory instructions are issued
    there, so vmcnt(N) covers the atomic;
  * in the basic block of every explicit wait, no instruction before the
    wait names a ticket register. That is where the compiler placed a copy
    of the register (`v_mov_b32 v2, v12` before `s_waitcnt vmcnt(0)`) when
    the wait statement took the ticket as an operand, a read of the register
    before the atomic had returned; the wait now takes no operands.
They also check that the library emits no buffer stores: a 16-byte buffer
store with a register scalar offset read its data registers after the next
VALU instruction had overwritten them on the MI355X (the compiler adds the
wait state after a global store of more than 8 bytes, and not after that
form), so full-tile stores are global stores.
"""
import os
import re
import shutil
import subprocess

import pytest

from dizo_amd import build as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNELS = os.path.join(ROOT, "dizo_amd", "csrc", "dz_kernels.hip")

VMEM = re.compile(r"^(global|buffer|flat|scratch)_(load|store|atomic)")


def _hipcc():
    try:
        return B.hipcc()
    except RuntimeError:
        return None


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    cc = _hipcc()
    if cc is None or shutil.which(cc) is None and not os.path.exists(cc):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "dz_kernels.s"
    flags = [f for f in B.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    subprocess.run([cc, *flags, "--cuda-device-only", "-S", KERNELS, "-o", str(out)], check=True,
                   capture_output=True, text=True)
    return out.read_text()


def _functions(text):
    """{name: [block, ...]} per kernel, a block being (label, [(instruction,
    in_inline_asm), ...]); fall-through blocks get the label of their comment
    (; %bb.N) or a synthetic one."""
    funcs, cur, blocks, inline = {}, None, None, False
    for raw in text.splitlines():
        if re.match(r"^_Z\S*:", raw):
            cur = raw.split(":")[0]
            blocks = funcs[cur] = [("entry", [])]
            inline = False
            continue
        if cur is None:
            continue
        if raw.startswith(".Lfunc_end"):
            cur = None
            continue
        s = raw.strip()
        m = re.match(r"^(\.LBB\w+):", raw) or re.match(r"^; (%bb\.\d+):", raw)
        if m:
            blocks.append((m.group(1), []))
            continue
        if s.startswith(";;#ASMSTART"):
            inline = True
            continue
        if s.startswith(";;#ASMEND"):
            inline = False
            continue
        s = s.split(";")[0].strip()
        if not s or s.startswith(".") or s.endswith(":"):
            continue
        blocks[-1][1].append((s, inline))
    return funcs


def _names_vgpr(ins: str, n: int) -> bool:
    ops = ins.split(None, 1)[1] if " " in ins else ""
    for m in re.finditer(r"\bv(\d+)\b|\bv\[(\d+):(\d+)\]", ops):
        if m.group(1) is not None and int(m.group(1)) == n:
            return True
        if m.group(2) is not None and int(m.group(2)) <= n <= int(m.group(3)):
            return True
    return False


def _is_ticket_wait(ins, inline):
    return inline and re.match(r"s_waitcnt vmcnt\(\d+\)$", ins)


ZERO_INIT = re.compile(r"v_mov_b(32|64)_e32 v(\d+|\[\d+:\d+\]), 0$")


def _ticket_pairs(funcs):
    for name, blocks in funcs.items():
        for b, (_, ins) in enumerate(blocks):
            for i, (text, inline) in enumerate(ins):
                m = re.match(r"global_atomic_add (v\d+), .*off sc0$", text)
                if inline and m:
                    yield name, int(m.group(1)[1:]), blocks, b, i


def _linear(blocks, b0, i0):
    """(instruction, inline, block index) from just after instruction i0 of
    block b0, in layout order."""
    for b in range(b0, len(blocks)):
        for k, (text, inline) in enumerate(blocks[b][1]):
            if b == b0 and k <= i0:
                continue
            yield text, inline, b


def test_every_ticket_has_a_wait_and_nothing_touches_its_register(asm):
    funcs = _functions(asm)
    pairs = list(_ticket_pairs(funcs))
    # the projection kernel's 15 instantiations (3 dtypes x 5 modes) take tickets this way
    assert len({p[0] for p in pairs}) >= 15, sorted({p[0] for p in pairs})
    tickets = {}
    for name, reg, blocks, b, i in pairs:
        tickets.setdefault(name, set()).add(reg)
        # (a) from the atomic to its first wait in layout order (the path the
        # compiler lays out straight after it), only the other paths'
        # zero-initialisation may name the register, and the wait counts no
        # more operations than that stretch issues
        nvm, waited = 0, None
        for text, inline, _ in _linear(blocks, b, i):
            if _is_ticket_wait(text, inline):
                waited = int(re.search(r"vmcnt\((\d+)\)", text).group(1))
                break
            assert not _names_vgpr(text, reg) or ZERO_INIT.match(text), (
                f"{name}: the ticket register v{reg} is used before its wait: {text}")
            nvm += bool(VMEM.match(text))
        assert waited is not None, f"{name}: ticket atomic into v{reg} has no explicit wait after it"
        assert waited == 0 or nvm >= waited, f"{name}: vmcnt({waited}) after only {nvm} vector-memory instructions"
    # (b) in the block of every explicit wait, nothing before the wait names a
    # ticket register (a copy placed there reads it before it has returned)
    for name, regs in tickets.items():
        for _, ins in funcs[name]:
            for k, (text, inline) in enumerate(ins):
                if not _is_ticket_wait(text, inline):
                    continue
                for prev, _ in ins[:k]:
                    for reg in regs:
                        assert not _names_vgpr(prev, reg) or ZERO_INIT.match(prev), (
                            f"{name}: v{reg} is used in the block of its wait, before it: {prev}")


def test_no_buffer_stores(asm):
    stores = [l.strip() for l in asm.splitlines() if re.match(r"\s*buffer_store", l)]
    assert not stores, stores[:3]


def test_names_vgpr_parser():
    assert _names_vgpr("v_mad_u64_u32 v[2:3], s[0:1], v5, s4, v[6:7]", 5)
    assert _names_vgpr("global_store_dwordx4 v[4:5], v[6:9], off nt", 8)
    assert not _names_vgpr("v_mov_b32_e32 v15, s3", 5)
    assert not _names_vgpr("v_add_u32_e32 v51, 0x400, v50", 5)
