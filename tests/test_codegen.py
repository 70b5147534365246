"""Static checks of the gfx950 code the kernel source compiles to (CPU only).

The K/V ring's barrier is a bare s_barrier (no memory fence), so the
property it relies on is checked on the generated code itself: at every
s_barrier of every entry, the wave has no LDS read in flight (an
``s_waitcnt lgkmcnt(0)`` follows the last ds_read).  A read left in flight
would race with the other waves' DMA refill of its stage right after the
barrier.  Also: no entry spills to scratch, every entry keeps two waves per
SIMD (the short form four), and no compiler-inserted wait holds a tile's
reads until the next tile's prefetch lands.
"""
import os
import re
import shutil
import subprocess

import pytest

from fmha_native_amd import build

_ENTRIES = [f"fmha_fwd_d64_bf16_{form}msk{m}{v}" for form in ("", "splitkv_", "pair_")
            for m in (0, 1) for v in ("", "_varlen")]


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if shutil.which(build.HIPCC) is None and not os.path.exists(build.HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "kernel.s"
    cmd = [build.HIPCC, *[f for f in build.HIP_FLAGS if f != "-fPIC"], "--cuda-device-only", "-S",
           os.path.join(build.CSRC, "fmha_fwd_kernel.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out.read_text()


def _functions(src):
    """Body of every function symbol (data symbols have labels too but no
    .Lfunc_end)."""
    funcs = {}
    for name in re.findall(r"^\s*\.type\s+(_Z[^,\s]+),@function", src, re.M):
        m = re.search(r"^" + re.escape(name) + r":", src, re.M)
        end = src.index(".Lfunc_end", m.end())
        funcs[name] = src[m.end():end]
    return funcs


def test_every_entry_compiled(asm):
    names = _functions(asm)
    for e in _ENTRIES:
        assert any(e + "13FmhaFwdParams" in n for n in names), e
    for e in ("fmha_fwd_d64_bf16_balanced_msk1", "fmha_fwd_d64_bf16_balanced_pair_msk1",
              "fmha_fwd_d64_bf16_balanced_merge", "fmha_fwd_d64_bf16_pair_stream_msk0",
              "fmha_fwd_d64_bf16_pair_stream_msk1", "fmha_fwd_d64_bf16_msk1_varlen_tilemajor",
              "fmha_fwd_d64_bf16_msk1_varlen_seqmajor"):
        assert any(e in n for n in names), e
    for m in (0, 1):
        for v in ("", "_varlen"):
            assert any(f"fmha_fwd_d64_bf16_short_msk{m}{v}13FmhaFwdParams" in n for n in names), (m, v)


def test_no_lds_read_in_flight_at_barriers(asm):
    for name, body in _functions(asm).items():
        pending, barriers = False, 0
        for line in body.splitlines():
            ins = line.strip()
            if ins.startswith("ds_read"):
                pending = True
            elif re.match(r"s_waitcnt\b.*lgkmcnt\(0\)", ins):
                pending = False
            elif ins.startswith("s_barrier"):
                barriers += 1
                assert not pending, f"{name}: LDS read in flight at barrier {barriers}"
        # every attention entry synchronises its K/V ring; the balanced form's
        # merge kernel has no ring (each wave stages its own rows)
        assert barriers > 0 or "balanced_merge" in name, name


def test_no_scratch_and_two_waves_per_simd(asm):
    scratch = re.findall(r"; ScratchSize: (\d+)", asm)
    occupancy = re.findall(r"; Occupancy: (\d+)", asm)
    assert scratch and all(int(s) == 0 for s in scratch), scratch
    assert occupancy and all(int(o) >= 2 for o in occupancy), occupancy


def _occupancy(src):
    """Occupancy (waves per SIMD) of every function from its kernel-info block."""
    occ = {}
    for m in re.finditer(r"^\s*\.set\s+(_Z[^.\s]+)\.has_indirect_call.*?; Occupancy: (\d+)", src, re.M | re.S):
        occ[m.group(1)] = int(m.group(2))
    return occ


def _lds_bytes(src):
    """LDS bytes per workgroup of every function from its kernel-info block."""
    lds = {}
    for m in re.finditer(r"^\s*\.set\s+(_Z[^.\s]+)\.has_indirect_call.*?; LDSByteSize: (\d+)", src, re.M | re.S):
        lds[m.group(1)] = int(m.group(2))
    return lds


def _prefetch_waits(body):
    """(wait, loads issued since the last barrier) for every vmcnt wait that
    precedes an LDS read with no barrier in between."""
    ins = [ln.strip() for ln in body.splitlines() if ln.strip() and not ln.strip().startswith((";", "."))]
    since, out = None, []
    for i, x in enumerate(ins):
        if x.startswith("s_barrier"):
            since = 0
        elif x.startswith("buffer_load") and since is not None:
            since += 1
        elif x.startswith("s_waitcnt") and "vmcnt" in x and since is not None:
            nxt = next((y for y in ins[i + 1:] if y.startswith(("s_barrier", "ds_read"))), "s_barrier")
            if nxt.startswith("ds_read"):
                out.append((int(re.search(r"vmcnt\((\d+)\)", x).group(1)), since))
    return out


def test_no_wait_covers_a_prefetch(asm):
    """Every entry prefetches K/V tiles by LDS-DMA right after a barrier and
    waits for them only before a later barrier.  Its ring stages are distinct
    LDS arrays indexed by compile-time stage numbers, so the compiler can
    tell that a prefetch does not alias the reads of the current tile; had it
    inserted a wait covering the prefetch before those reads, every tile
    would wait for the next one's loads.  So a vmcnt wait that precedes an
    LDS read (no barrier in between) must let every load issued since the
    last barrier stay in flight (the compiler adds such waits for register
    loads such as Q: it does not see the hand-written waits)."""
    for name, body in _functions(asm).items():
        for n, since in _prefetch_waits(body):
            assert n >= since, (name, n, since)


def test_short_entries(asm):
    """The short entries' prologue issues K(0) and V(0) into LDS and Q into
    registers (two, two and four loads per wave) before the first barrier,
    and their loop waits with the s_waitcnt builtin, which the compiler's own
    wait placement sees: it adds no wait between a prefetch and the tile's
    LDS reads at all (with an inline-asm wait it did, one that also covered
    the conditional prefetch).  32 KiB of LDS and <= 128 VGPRs keep four
    blocks per compute unit."""
    occ, lds = _occupancy(asm), _lds_bytes(asm)
    rings = {n: b for n, b in _functions(asm).items() if "_short_msk" in n}
    assert len(rings) == 4
    for name, body in rings.items():
        assert occ.get(name) == 4, (name, occ.get(name))
        assert lds.get(name) == 32 * 1024, (name, lds.get(name))
        ins = [ln.strip() for ln in body.splitlines() if ln.strip() and not ln.strip().startswith((";", "."))]
        first = next(i for i, x in enumerate(ins) if x.startswith("s_barrier"))
        loads = [x for x in ins[:first] if x.startswith("buffer_load_dwordx4")]
        assert sorted("L" if x.endswith(" lds") else "R" for x in loads) == ["L"] * 4 + ["R"] * 4, (name, loads)
        assert all(since == 0 for _, since in _prefetch_waits(body)), name
