"""Static check of the gfx950 code of every kernel entry (CPU only): no
instruction reads an SGPR that held a preloaded workgroup id while an
undefined value (an ``implicit-def`` in the compiler's listing) can reach it
along some path.

A build of the causal entries that branched on the grid's shape before
reading blockIdx.z had such a path: the register holding blockIdx.z was
reused for gridDim.y inside the branch, and on the path that fell through
the batch index was taken from it, so batch-1 launches addressed batch
gridDim.y.  The LLVM IR was correct there; only the listing shows it, as an
implicit-def of the id registers on that path.  The entries now take every
index straight from a grid coordinate; this test keeps any entry from
reintroducing the pattern unnoticed.

The check is a forward dataflow over the listing's basic blocks (labels and
branches): each id register holds the id at entry and an ordinary value once
an instruction writes it; an implicit-def is reported where the register may
still hold the id on some path reaching it (the faulting build's case: its
implicit-def sat on the path where the register was never written).  An
implicit-def after the register was overwritten on every path concerns an
ordinary value (an entry that copies an id out in its first instruction may
reuse the register).
"""
import os
import re
import shutil
import subprocess

import pytest

from fmha_native_amd import build

_SOURCES = ["fmha_fwd_kernel.hip", "fmha_merge.hip"]


def _device_asm(tmp_path, name):
    out = tmp_path / (name + ".s")
    cmd = [build.HIPCC, *[f for f in build.HIP_FLAGS if f != "-fPIC"], "--cuda-device-only", "-S",
           os.path.join(build.CSRC, name), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out.read_text()


def id_registers(asm):
    """{kernel symbol: [SGPR numbers holding workgroup id x, y, z]} from the
    kernel descriptors: the ids follow the user SGPRs, in x, y, z order, one
    register for each id the descriptor enables."""
    out = {}
    for m in re.finditer(r"^\s*\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", asm, re.M | re.S):
        body = m.group(2)
        first = int(re.search(r"\.amdhsa_user_sgpr_count (\d+)", body).group(1))
        regs = []
        for axis in "xyz":
            hit = re.search(rf"\.amdhsa_system_sgpr_workgroup_id_{axis} (\d)", body)
            if hit and hit.group(1) == "1":
                regs.append(first + len(regs))
        out[m.group(1)] = regs
    return out


# mnemonics whose first operand is not a destination SGPR (VALU, DS and memory
# instructions' first operands are VGPRs or SGPR destinations, both fine here)
_NO_SGPR_DEST = re.compile(r"^(s_cmp|s_bitcmp|s_waitcnt|s_barrier|s_nop|s_branch|s_cbranch|s_setprio|s_sleep|"
                           r"s_endpgm|s_sendmsg|s_trap|s_dcache|s_icache|s_ttrace|s_set_gpr|s_sethalt)")


def _sgprs(operand):
    """SGPR numbers named by one operand: s7 or s[4:5]."""
    m = re.fullmatch(r"s(\d+)", operand)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", operand)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def _instructions(body):
    """[(kind, payload)] per listing line: ('label', name), ('undef', {regs}),
    ('ins', (mnemonic, [operands]))."""
    out = []
    for line in body.splitlines():
        t = line.strip()
        m = re.match(r"^(\.LBB\d+_\d+):", t)
        if m:
            out.append(("label", m.group(1)))
            continue
        m = re.search(r"implicit-def: (.*)$", t)
        if m and t.startswith(";"):
            out.append(("undef", {int(r) for r in re.findall(r"\$sgpr(\d+)\b(?!_)", m.group(1))}))
            continue
        if not t or t.startswith((";", ".")):
            continue
        t = t.split(";")[0].strip()
        mn, _, rest = t.partition(" ")
        ops = [o.strip() for o in re.split(r",(?![^\[]*\])", rest) if o.strip()]
        out.append(("ins", (mn, ops)))
    return out


_TERMINATORS = ("s_branch", "s_setpc", "s_endpgm", "s_trap")


def id_killing_undefs(body, regs):
    """Id registers in `regs` given an implicit-def at a point that the id can
    reach unwritten (forward dataflow over the basic blocks of one body)."""
    blocks, labels, cur = [], {}, []
    for kind, pay in _instructions(body):
        if kind == "label":
            if cur:
                blocks.append(cur)
            cur = []
            labels[pay] = len(blocks)
            continue
        cur.append((kind, pay))
        if kind == "ins" and (pay[0].startswith("s_cbranch") or pay[0].startswith(_TERMINATORS)):
            blocks.append(cur)
            cur = []
    blocks.append(cur)
    succ = []
    for i, blk in enumerate(blocks):
        out = set()
        last = blk[-1][1] if blk and blk[-1][0] == "ins" else None
        if last and (last[0].startswith("s_branch") or last[0].startswith("s_cbranch")) and last[1]:
            if last[1][0] in labels:
                out.add(labels[last[1][0]])
        if not (last and last[0].startswith(_TERMINATORS)) and i + 1 < len(blocks):
            out.add(i + 1)
        succ.append(out)
    # holds_id[i]: id registers that may still hold the id entering block i
    holds_id = [set() for _ in blocks]
    holds_id[0] = set(regs)
    bad, work = set(), [0]
    while work:
        i = work.pop()
        live = set(holds_id[i])
        for kind, pay in blocks[i]:
            if kind == "undef":
                bad |= live & pay
                live -= pay
            elif kind == "ins":
                mn, ops = pay
                if ops and not _NO_SGPR_DEST.match(mn):
                    live -= _sgprs(ops[0])
        for j in succ[i]:
            if not live <= holds_id[j]:
                holds_id[j] |= live
                work.append(j)
    return sorted(bad)


def undefined_id_registers(asm):
    """{kernel symbol: sorted id registers given an implicit-def while they
    may still hold the id}"""
    bad = {}
    for name, regs in id_registers(asm).items():
        start = re.search(rf"^{re.escape(name)}:", asm, re.M)
        end = asm.index(".Lfunc_end", start.end())
        hit = id_killing_undefs(asm[start.end():end], regs)
        if hit:
            bad[name] = hit
    return bad


@pytest.mark.parametrize("name", _SOURCES)
def test_workgroup_id_registers_never_undefined(tmp_path, name):
    if shutil.which(build.HIPCC) is None and not os.path.exists(build.HIPCC):
        pytest.skip("hipcc not available")
    asm = _device_asm(tmp_path, name)
    ids = id_registers(asm)
    assert ids and all(ids.values()), "no kernel descriptors found"
    assert undefined_id_registers(asm) == {}


def test_checker_sees_an_undefined_id_register():
    # a listing shaped like the faulting build's: ids in s2..s4 after two user
    # SGPRs; one path loads gridDim.y into s4 (blockIdx.z), the other marks it
    # undefined, and the join reads s4 as the batch index
    listing = """k:
	s_cmp_eq_u32 s3, 0
	s_cbranch_scc1 .LBB0_19
	s_load_dword s4, s[6:7], 0x14
	s_branch .LBB0_6
.LBB0_19:
                                        ; implicit-def: $sgpr4
	s_branch .LBB0_6
.LBB0_6:
	s_mul_i32 s8, s4, s9
	s_endpgm
.Lfunc_end0:
	.amdhsa_kernel k
		.amdhsa_user_sgpr_count 2
		.amdhsa_system_sgpr_workgroup_id_x 1
		.amdhsa_system_sgpr_workgroup_id_y 1
		.amdhsa_system_sgpr_workgroup_id_z 1
	.end_amdhsa_kernel
"""
    assert id_registers(listing) == {"k": [2, 3, 4]}
    assert undefined_id_registers(listing) == {"k": [4]}
    assert undefined_id_registers(listing.replace("$sgpr4", "$sgpr40")) == {}
    # copying the id out and overwriting the register on every path before an
    # implicit-def is fine; the faulting build's implicit-def sat on the path
    # where the register still held the id
    copied = listing.replace("\ts_cmp_eq_u32 s3, 0", "\ts_mov_b32 s40, s4\n\ts_mov_b32 s4, 7\n\ts_cmp_eq_u32 s3, 0")
    assert undefined_id_registers(copied) == {}
    late = listing.replace("; implicit-def: $sgpr4\n\ts_branch .LBB0_6",
                           "s_mov_b32 s4, 1\n; implicit-def: $sgpr4\n\ts_branch .LBB0_6")
    assert undefined_id_registers(late) == {}
