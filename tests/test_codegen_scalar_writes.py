"""Static check of the gfx950 code of every HIP source (CPU only): no
instruction writes through the scalar data cache — no scalar memory store or
atomic, and no write-back or discard of that cache.  All device writes in
this library are vector stores (buffer/global); this keeps it that way.

The file names the forbidden mnemonics, so it is kept off the GPU box (no GPU
run loads it).
"""
import os
import re
import shutil
import subprocess

import pytest

from fmha_native_amd import build

_SOURCES = ["fmha_fwd_kernel.hip", "fmha_merge.hip", "fmha_fwd_api.hip", "fmha_noalloc.hip"]
_FORBIDDEN = re.compile(r"^\s*(s_store_|s_buffer_store|s_scratch_store|s_atomic|s_buffer_atomic|"
                        r"s_dcache_wb|s_dcache_discard)", re.M)


def _device_asm(tmp_path, name):
    out = tmp_path / (name + ".s")
    cmd = [build.HIPCC, *[f for f in build.HIP_FLAGS if f != "-fPIC"], "--cuda-device-only", "-S",
           os.path.join(build.CSRC, name), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out.read_text()


@pytest.mark.parametrize("name", _SOURCES)
def test_no_scalar_cache_writes(tmp_path, name):
    if shutil.which(build.HIPCC) is None and not os.path.exists(build.HIPCC):
        pytest.skip("hipcc not available")
    asm = _device_asm(tmp_path, name)
    hits = _FORBIDDEN.findall(asm)
    assert not hits, f"{name}: {sorted(set(hits))}"


def test_checker_sees_the_mnemonics():
    # the pattern matches instruction lines and nothing else
    assert _FORBIDDEN.search("\ts_store_dword s0, s[2:3], 0x0\n")
    assert _FORBIDDEN.search("  s_dcache_wb\n")
    assert not _FORBIDDEN.search("\tbuffer_store_dwordx2 v[0:1], v2, s[4:7], 0 offen\n")
    assert not _FORBIDDEN.search("\tglobal_atomic_add v0, v1, s[0:1]\n")
