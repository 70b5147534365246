"""Static check of the gfx950 code of every kernel entry (CPU only): the SGPRs
that hold the preloaded workgroup ids never receive an undefined value (an
``implicit-def`` in the compiler's listing) on any path.

A build of the causal entries that branched on the grid's shape before
reading blockIdx.z had such a path: the register holding blockIdx.z was
reused for gridDim.y inside the branch, and on the path that fell through
the batch index was taken from it, so batch-1 launches addressed batch
gridDim.y.  The LLVM IR was correct there; only the listing shows it, as an
implicit-def of the id registers on that path.  The entries now take every
index straight from a grid coordinate; this test keeps any entry from
reintroducing the pattern unnoticed.
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


def undefined_id_registers(asm):
    """{kernel symbol: sorted id registers the listing gives an implicit-def}"""
    bad = {}
    for name, regs in id_registers(asm).items():
        start = re.search(rf"^{re.escape(name)}:", asm, re.M)
        end = asm.index(".Lfunc_end", start.end())
        defs = {int(r) for r in re.findall(r"implicit-def: \$sgpr(\d+)\b(?!_)", asm[start.end():end])}
        hit = sorted(defs & set(regs))
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
    # SGPRs, and a path that marks s4 (blockIdx.z) undefined
    listing = """k:
	s_load_dword s4, s[6:7], 0x14
.LBB0_19:
                                        ; implicit-def: $sgpr4
	s_branch .LBB0_6
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
