"""The drop-in boundary without a GPU: the C-ABI library loads, exports every
symbol include/*.h declares, the kernarg layout matches the reference's struct
byte for byte (src/runner/params.hpp:18-64, offsets measured from the C
header by a gcc-compiled probe), and the launcher's argument checks return the
documented hipError_t codes.  No HIP call that needs a device is made.
"""
import ctypes
import os
import re
import subprocess
import sys
import tempfile

import numpy as np
import pytest

import fmha_native_amd as fmha

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")

# the reference struct's field offsets (src/runner/params.hpp:18-64)
REFERENCE_OFFSETS = {
    "q": 0, "k": 8, "v": 16, "o": 24, "lse": 32, "seqlen_q": 40, "seqlen_k": 44, "nhead_q": 48, "nhead_k": 52,
    "scale": 56, "stride_q": 60, "nhead_stride_q": 64, "batch_stride_q": 68, "stride_k": 72,
    "nhead_stride_k": 76, "batch_stride_k": 80, "stride_v": 84, "nhead_stride_v": 88, "batch_stride_v": 92,
    "stride_o": 96, "nhead_stride_o": 100, "batch_stride_o": 104, "seqstart_q": 112, "seqstart_k": 120,
}
KERNEL_ENTRIES = ["fmha_fwd_d64_bf16_msk0", "fmha_fwd_d64_bf16_msk1", "fmha_fwd_d64_bf16_msk0_varlen",
                  "fmha_fwd_d64_bf16_msk1_varlen"]
SPLIT_ENTRIES = [f"fmha_fwd_d64_bf16_{form}_msk{m}{v}" for form in ("splitkv", "pair") for m in (0, 1)
                 for v in ("", "_varlen")] + [f"fmha_fwd_d64_bf16_{f}msk1_tilemajor" for f in ("", "splitkv_", "pair_")] \
    + [f"fmha_fwd_d64_bf16_short_msk{m}{v}" for m in (0, 1) for v in ("", "_varlen")] \
    + ["fmha_fwd_d64_bf16_msk1_varlen_tilemajor", "fmha_fwd_d64_bf16_msk1_varlen_seqmajor"]


def header_c_functions():
    """Names of the functions declared inside extern "C" blocks of include/*.h."""
    names = []
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"^\s*#.*$", "", text, flags=re.M)  # preprocessor lines (macro values in parentheses)
        text = re.sub(r"typedef struct.*?\}\s*\w+\s*;", "", text, flags=re.S)
        for block in re.findall(r'extern "C" \{(.*?)\n\}', text, flags=re.S):
            names += re.findall(r"\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*;", block)
    return names


def exported_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_loads_and_exports_header_symbols():
    lib = fmha.load_library()
    names = header_c_functions()
    assert {"fmha_fwd_d64_bf16", "fmha_fwd_d64_bf16_check", "fmha_fwd_d64_bf16_tile_config"} <= set(names)
    syms = exported_symbols(fmha.LIB_PATH)
    for n in names:
        assert n in syms, n
        assert getattr(lib, n) is not None


def test_kernel_entries_exported():
    """The four __global__ entries keep the reference's C++ names
    (src/fused/kernel.cpp:55-99), so its callers link unchanged."""
    syms = exported_symbols(fmha.LIB_PATH)
    for e in KERNEL_ENTRIES + SPLIT_ENTRIES:
        mangled = f"_Z{len(e)}{e}13FmhaFwdParams"
        assert mangled in syms, mangled


def test_ctypes_layout_matches_reference():
    assert ctypes.sizeof(fmha.FmhaFwdParams) == 128
    assert ctypes.alignment(fmha.FmhaFwdParams) == 8
    for name, off in REFERENCE_OFFSETS.items():
        assert getattr(fmha.FmhaFwdParams, name).offset == off, name


def test_c_header_layout_matches_reference():
    """Compile include/fmha_fwd.h as plain C with gcc and print every offsetof."""
    fields = list(REFERENCE_OFFSETS)
    src = "#include <stdio.h>\n#include <stddef.h>\n#include \"fmha_fwd.h\"\nint main(void){\n"
    src += 'printf("%zu %zu\\n", sizeof(FmhaFwdParams), _Alignof(FmhaFwdParams));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof(FmhaFwdParams, {f}));\n'
    src += "return 0;}\n"
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "probe.c")
        exe = os.path.join(d, "probe")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", f"-I{INCLUDE}", "-I/opt/rocm/include", c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()
    assert out[0] == "128" and out[1] == "8"
    assert [int(x) for x in out[2:]] == [REFERENCE_OFFSETS[f] for f in fields]


def test_tile_config():
    assert fmha.tile_config() == {"kM0": 128, "kN0": 64, "kBlockSize": 256, "kHeadDim": 64}


def test_missing_library_raises():
    import importlib

    mod = importlib.import_module("fmha_native_amd")
    saved = mod._lib
    try:
        mod._lib = None
        with pytest.raises(FileNotFoundError):
            mod.load_library(os.path.join(ROOT, "does_not_exist.so"))
    finally:
        mod._lib = saved


# ---------------------------------------------------------------- argument checks

def valid_params(varlen=False, lse=True):
    p = fmha.FmhaFwdParams()
    base = 0x10000
    p.q, p.k, p.v, p.o = base, base + 0x1000, base + 0x2000, base + 0x3000
    p.lse = base + 0x4000 if lse else None
    p.seqlen_q = p.seqlen_k = 128
    p.nhead_q, p.nhead_k = 4, 2
    p.scale = fmha.LOG2E / 8
    for t in "qkvo":
        setattr(p, f"stride_{t}", 64)
        setattr(p, f"nhead_stride_{t}", 128 * 64)
        setattr(p, f"batch_stride_{t}", 4 * 128 * 64)
    if varlen:
        p.seqstart_q = p.seqstart_k = base + 0x5000
    return p


INVALID = 1  # hipErrorInvalidValue


@pytest.mark.parametrize("varlen", [False, True])
def test_check_accepts_valid(varlen):
    assert fmha.check_params(valid_params(varlen), 2, 0) == 0
    assert fmha.check_params(valid_params(varlen), 2, 1) == 0
    assert fmha.check_params(valid_params(varlen, lse=False), 0, 1) == 0


def _mut(**kw):
    p = valid_params(kw.pop("varlen", False))
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("params,batch,causal", [
    (_mut(q=None), 1, 0),
    (_mut(o=None), 1, 0),
    (_mut(k=0x10002), 1, 0),                 # not 16-byte aligned
    (_mut(lse=0x10002), 1, 0),               # LSE not 4-byte aligned
    (_mut(stride_q=60), 1, 0),               # stride not a multiple of 8 (16-byte rows)
    (_mut(stride_v=56), 1, 0),               # row shorter than 64 elements
    (_mut(nhead_stride_k=-64), 1, 0),
    (_mut(seqlen_q=-1), 1, 0),
    (_mut(scale=0.0), 1, 0),                 # the running max needs a positive scale
    (_mut(scale=-0.18), 1, 0),
    (_mut(scale=float("nan")), 1, 0),
    (_mut(scale=float("inf")), 1, 0),
    (_mut(seqlen_k=16_776_894), 1, 0),       # one row past the 31-bit offset bound (rows + 320 rows of headroom)
    (_mut(nhead_k=3), 1, 0),                 # nhead_q % nhead_k != 0
    (_mut(nhead_k=0), 1, 0),
    (_mut(seqstart_q=0x15000), 1, 0),        # only one seqstart pointer
    (_mut(stride_k=1 << 23), 1, 0),          # offsets beyond 31 bits
    (_mut(varlen=True, nhead_stride_q=128 * 64 + 8), 1, 0),  # varlen LSE head stride not in rows
    (_mut(seqlen_q=65535 * 128 + 1, lse=None), 1, 0),  # grid y = ceil(seqlen_q / 128) above 65535
    (valid_params(), 65536, 0),                          # grid z = batch above 65535
    (valid_params(), -1, 0),
    (valid_params(), 1, 2),
])
def test_check_rejects(params, batch, causal):
    assert fmha.check_params(params, batch, causal) == INVALID


def test_offset_bound_edge():
    """The last row count the 31-bit offset check accepts for 64-element rows:
    (rows + 64 + 256) * 128 bytes + 256 < 2^31."""
    assert fmha.check_params(_mut(seqlen_k=16_776_893), 1, 0) == 0
    assert fmha.check_params(_mut(seqlen_k=16_776_894), 1, 0) == INVALID
    # Q and O: the same bound with a wider row stride (grid y caps seqlen_q first otherwise)
    assert fmha.check_params(_mut(seqlen_q=8_388_286, stride_q=128), 1, 0) == 0
    assert fmha.check_params(_mut(seqlen_q=8_388_287, stride_q=128), 1, 0) == INVALID


def test_variant_validation():
    """An unknown kernel form is rejected before anything is launched."""
    lib = fmha.load_library()
    p = valid_params()
    # 0-3, 6 and 8 are the valid forms, optionally OR-ed with one order flag
    # (VARIANT_REFERENCE_ORDER 16, VARIANT_TILE_MAJOR_ORDER 32, VARIANT_SEQUENCE_ORDER 64); 4 is retired,
    # 5 and 7 (the balanced forms) need the workspace entry; two order flags at once are rejected
    R, T, S = fmha.VARIANT_REFERENCE_ORDER, fmha.VARIANT_TILE_MAJOR_ORDER, fmha.VARIANT_SEQUENCE_ORDER
    for bad in (-1, 4, 5, 7, 9, 100, 128, R | 7, T | 4, R | T, T | S, R | S, R | T | S, R | T | 1):
        assert lib.fmha_fwd_d64_bf16_variant(ctypes.byref(p), 1, 0, bad, None) == INVALID, bad
    for bad in (R | T, T | S | 2):
        assert lib.fmha_fwd_d64_bf16_ws(ctypes.byref(p), 1, 1, bad, None, 0, None) == INVALID, bad
        assert lib.fmha_fwd_d64_bf16_workspace_size(ctypes.byref(p), 1, 1, bad) == -1, bad
    bad_p = _mut(q=None)
    assert lib.fmha_fwd_d64_bf16_variant(ctypes.byref(bad_p), 1, 0, fmha.VARIANT_SPLITKV, None) == INVALID


def test_null_params_pointer():
    lib = fmha.load_library()
    assert lib.fmha_fwd_d64_bf16_check(None, 1, 0) == INVALID


# ---------------------------------------------------------------- kernel-form policy

def _shape(batch, heads, seqlen):
    p = valid_params(lse=False)
    p.nhead_q = p.nhead_k = heads
    p.seqlen_q = p.seqlen_k = seqlen
    return p, batch


R, S, P = fmha.VARIANT_REGULAR, fmha.VARIANT_SPLITKV, fmha.VARIANT_PAIR


def test_short_form_rule():
    """Launches whose keys fit three 64-key tiles take the short form once
    they hold two blocks' worth of query rows per compute unit (2 x CUs x 128
    rows), causal ones with up to 384 keys once they hold seven; varlen ones
    by their bounds (batch x nhead_q x seqlen_q rows, seqlen_k keys: the
    short form reads each sequence's own lengths, so the bounds only steer
    the choice); smaller grids keep the grid-shape rule."""
    # valid_params: 4 heads x 128 query rows per batch -> 512 rows
    for sk, batch, cus, dense, causal_short in (
            (1, 128, 256, True, True), (64, 128, 256, True, True), (128, 128, 256, True, True),
            (128, 127, 256, False, False), (128, 152, 304, True, True), (128, 151, 304, False, False),
            (128, 4096, 256, True, True),
            (129, 128, 256, True, True), (192, 128, 256, True, True), (192, 127, 256, False, False),
            (193, 447, 256, False, False), (193, 448, 256, False, True), (384, 448, 256, False, True),
            (384, 531, 304, False, False), (384, 532, 304, False, True), (385, 4096, 256, False, False),
            (513, 4096, 256, False, False), (2048, 4096, 256, False, False)):
        for causal, short in ((0, dense), (1, causal_short)):
            got = fmha.pick_variant(_mut(seqlen_k=sk, lse=None), batch, causal, cus)
            assert (got == fmha.VARIANT_SHORT) if short else (got in (R, S, P)), (sk, batch, cus, causal, got)
    # varlen: valid_params bounds 128 keys and 128 query rows per sequence, 4 heads
    pv = valid_params(varlen=True, lse=False)
    assert fmha.pick_variant(pv, 4096, 1, 256) == fmha.VARIANT_SHORT
    assert fmha.pick_variant(pv, 127, 1, 256) in (R, S, P)
    pv.seqlen_k = 4096
    assert fmha.pick_variant(pv, 4096, 1, 256) in (R, S, P)


@pytest.mark.parametrize("batch,heads,seqlen,causal,cus,form", [
    (1, 8, 4096, 0, 256, S),     # 256 blocks: at most one per CU
    (1, 2, 4096, 0, 256, S),     # 64 blocks
    (1, 32, 1024, 0, 256, R),    # 256 blocks, but 1024 keys: halves too short
    (1, 64, 512, 1, 256, R),
    (1, 2, 256, 0, 256, R),      # 4 blocks, 4 key tiles
    (1, 2, 2048, 1, 256, S),     # 2048 keys: split
    (1, 12, 4096, 0, 256, R),    # 384 dense blocks
    (1, 12, 4096, 1, 256, S),    # 384 causal blocks = 1.5 per CU: still split
    (1, 13, 4096, 1, 256, R),    # 416 causal blocks, short M-tiles
    (1, 8, 8192, 1, 256, S),     # 512 causal blocks with seqlen_k >= 8192
    (1, 32, 2048, 1, 256, R),    # 512 causal blocks, short M-tiles
    (4, 16, 2048, 0, 256, P),    # cfg2: 512 pair blocks = 2 whole rounds
    (1, 16, 8192, 1, 256, P),    # cfg3: 512 causal pair blocks = exactly 2 rounds
    (1, 8, 8192, 0, 256, P),     # 256 pair blocks, long M-tiles
    (1, 4, 32768, 1, 256, P),    # 512 causal pair blocks, seqlen_k >= 32768
    (1, 8, 32768, 1, 256, P),    # 1024 causal pair blocks (4 rounds), seqlen_k >= 32768
    (1, 32, 8192, 1, 256, R),    # 1024 causal pair blocks (4 rounds) below 32768 keys
    (1, 24, 8192, 1, 256, R),    # 768 causal pair blocks (3 rounds)
    (2, 16, 4096, 1, 256, R),    # 2 causal rounds but seqlen_k < 8192
    (4, 16, 2048, 1, 256, R),    # causal S2048
    (1, 32, 2048, 0, 256, P),    # 256 dense pair blocks (1 round) at 2048 keys
    (8, 16, 1024, 0, 256, R),    # dense, whole rounds, but 1024 keys
    (5, 16, 2048, 0, 256, R),    # 640 dense pair blocks: a partial last round
    (1, 2, 40000, 0, 256, R),    # 314 pair blocks: a partial last round
    (1, 2, 40000, 1, 256, R),    # cfg5
    (1, 8, 4096, 0, 304, S),     # the rule scales with the CU count
    (4, 16, 2048, 0, 304, R),    # 512 pair blocks: not whole rounds of 304
    (1, 19, 8192, 0, 304, P),    # 19 * 32 = 608 pair blocks = 2 rounds of 304
    (1, 19, 8192, 1, 304, P),    # the same, causal: exactly 2 rounds
])
def test_auto_form_rule(batch, heads, seqlen, causal, cus, form):
    """The launcher's documented rule (grid shape -> kernel form), host only."""
    p, b = _shape(batch, heads, seqlen)
    assert fmha.pick_variant(p, b, causal, cus) == form


@pytest.mark.parametrize("batch,heads,kv_heads,seqlen,causal,varlen,expect", [
    (8, 16, 16, 1024, 1, False, 1),    # 8 x 2 x 1024 x 256 B = 4 MiB per XCD
    (4, 16, 16, 2048, 1, False, 1),    # 4 MiB
    (16, 8, 8, 2048, 1, False, 1),     # 8 MiB: the limit itself
    (16, 16, 16, 2048, 1, False, 0),   # 16 MiB
    (4, 32, 32, 4096, 1, False, 0),    # 16 MiB
    (16, 16, 2, 2048, 1, False, 1),    # GQA: 2 K/V heads are at most one per XCD -> 8 MiB
    (17, 16, 2, 2048, 1, False, 0),    # 8.5 MiB
    (1, 16, 16, 8192, 1, False, 0),    # one batch: nothing to interleave
    (8, 16, 16, 1024, 0, False, 0),    # dense: every block costs the same
    (8, 16, 16, 1024, 1, True, 2),     # varlen causal, <= 8 sequences, grid 1024 <= 16 x 256: sequence order
    (8, 16, 16, 4096, 1, True, 2),     # grid 4096 = 16 x 256 (cfg4's bound is 3968)
    (8, 16, 16, 4224, 1, True, 0),     # grid 4224 > 16 x 256: the reference's order
    (9, 16, 16, 1024, 1, True, 0),     # more than 8 sequences: the reference's order
    (8, 16, 16, 1024, 0, True, 0),     # varlen dense: the reference's order
    (1, 8, 8, 4096, 1, True, 0),       # the split-KV form keeps the reference's order
    (8, 64, 64, 128, 1, True, 0),      # so does the short form
])
def test_tile_major_rule(batch, heads, kv_heads, seqlen, causal, varlen, expect):
    """Causal dense batches run tile-major while the K/V one XCD serves,
    batch x ceil(nhead_k/8) x seqlen_k x 256 bytes, is at most 8 MiB (1);
    causal varlen launches in the regular form of at most 8 sequences on a
    grid of at most 16 x CUs blocks run the sequence order (2)."""
    p = valid_params(lse=False)
    p.nhead_q, p.nhead_k = heads, kv_heads
    p.seqlen_q = p.seqlen_k = seqlen
    if varlen:
        seq = (ctypes.c_int32 * 2)(0, seqlen)
        p.seqstart_q = p.seqstart_k = ctypes.cast(seq, ctypes.c_void_p).value
    assert fmha.tile_major(p, batch, causal) == expect


def test_rules_at_extreme_counts():
    """Head and CU counts near INT_MAX: the rules stay defined and monotone."""
    big = 2**31 - 1
    p = valid_params(lse=False)
    p.nhead_q = p.nhead_k = big
    p.seqlen_k = 600  # past the short form's 384 keys
    assert fmha.tile_major(p, 65535, 1) == 0
    assert fmha.pick_variant(p, 65535, 1, 256) == R
    q = valid_params(lse=False)
    q.seqlen_q = q.seqlen_k = 4096                    # long enough for the split-KV form
    assert fmha.pick_variant(q, 1, 1, big) == S       # every grid fits such a device at once
    q.seqlen_k = 0
    assert fmha.tile_major(q, 65535, 1) == 1          # no K/V at all


def test_tile_major_only_when_something_is_launched():
    p = valid_params(lse=False)
    p.seqlen_q = 0
    assert fmha.tile_major(p, 4, 1) == 0


def test_tile_major_rejects_what_the_launch_rejects():
    assert fmha.tile_major(_mut(q=None), 2, 1) == -1
    assert fmha.tile_major(valid_params(), 2, 2) == -1


def test_auto_form_rejects_what_the_launch_rejects():
    assert fmha.pick_variant(_mut(q=None), 1, 0, 256) == -1
    assert fmha.pick_variant(valid_params(), 1, 2, 256) == -1
    assert fmha.pick_variant(valid_params(), 1, 0, -1) == -1
    assert fmha.pick_variant(valid_params(), 4096, 0) == fmha.VARIANT_SHORT  # 128 keys, 2M query rows
    assert fmha.pick_variant(_mut(seqlen_k=129), 1, 0) in (R, S, P)  # the current device's count


# ---------------------------------------------------------------- bench contract

def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


# ---------------------------------------------------------------- balanced causal form (host only)

def _ntiles(mt, sq, sk):
    last = min(mt * 128 + 127, sq - 1)
    e = max(0, min(sk, last + (sk - sq) + 1))
    return (e + 63) // 64


@pytest.mark.parametrize("b,h,sq,sk,cus,force", [
    (1, 2, 40000, 40000, 256, False),   # cfg5: heavy M-tiles
    (1, 2, 40000, 40000, 304, False),
    (2, 3, 3000, 3500, 256, True),
    (1, 1, 300, 200, 256, True),
])
def test_balanced_plan_is_longest_first_over_every_key_tile(b, h, sq, sk, cus, force):
    """The plan covers every key tile of every M-tile exactly once (whole
    M-tiles below split_from, two halves from it on), in non-increasing order
    of work, and splits exactly the M-tiles with more key tiles than half the
    average work per resident block (two blocks per compute unit)."""
    p = valid_params(lse=False)
    p.nhead_q, p.nhead_k, p.seqlen_q, p.seqlen_k = h, h, sq, sk
    items, sf = fmha.balanced_plan(p, b, 1, cus, force, xccs=1)  # the plain order
    m_tiles = -(-sq // 128)
    n = [_ntiles(mt, sq, sk) for mt in range(m_tiles)]
    avg = sum(n) * h * b / (2 * cus)
    assert sf == sum(1 for x in n if x <= max(2.0, avg / 2))
    expect = {(mt, None) for mt in range(sf)} | {(mt, half) for mt in range(sf, m_tiles) for half in (0, 1)}
    assert len(items) == len(expect) and set(items) == expect
    work = [n[mt] if half is None else (n[mt] + 1) // 2 if half == 0 else n[mt] // 2 for mt, half in items]
    assert all(x >= y for x, y in zip(work, work[1:]))
    ws = fmha.workspace_size(p, b, 1, fmha.VARIANT_BALANCED if force else fmha.VARIANT_AUTO) if cus == 256 else None
    if ws is not None:
        assert ws == (m_tiles - sf) * h * b * 2 * 4 * 34 * 64 * 4


@pytest.mark.parametrize("b,h,sq,sk,cus", [
    (1, 2, 40000, 40000, 256),   # cfg5: 313 M-tiles, an odd last pair
    (1, 2, 40064, 40064, 256),   # 313 M-tiles, the last one full
    (2, 3, 3000, 3500, 256),
    (1, 1, 300, 200, 256),       # one pair, not split
    (1, 4, 8192, 8192, 64),
])
def test_balanced_pair_plan_covers_every_pair_once(b, h, sq, sk, cus):
    """The plan over M-tile pairs (one 8-wave block per compute unit): unit u
    is M-tiles 2u and 2u+1 with the key tiles of the later one; whole units
    below split_from / 2 and two halves from it on, in non-increasing order
    of work; split_from is even (both M-tiles of a split pair are split) or
    the M-tile count; the workspace holds two partials per split M-tile."""
    p = valid_params(lse=False)
    p.nhead_q, p.nhead_k, p.seqlen_q, p.seqlen_k = h, h, sq, sk
    items, sf = fmha.balanced_plan(p, b, 1, cus, "pair", xccs=1)  # the plain order
    m_tiles = -(-sq // 128)
    units = (m_tiles + 1) // 2
    n = [_ntiles(min(2 * u + 1, m_tiles - 1), sq, sk) for u in range(units)]
    avg = sum(n) * h * b / cus
    su = sum(1 for x in n if x <= max(2.0, 0.7 * avg))
    assert all(x <= y for x, y in zip(n, n[1:]))
    assert sf == min(2 * su, m_tiles) and (sf % 2 == 0 or sf == m_tiles)
    expect = {(u, None) for u in range(su)} | {(u, half) for u in range(su, units) for half in (0, 1)}
    assert len(items) == len(expect) and set(items) == expect
    work = [n[u] if half is None else (n[u] + 1) // 2 if half == 0 else n[u] // 2 for u, half in items]
    assert all(x >= y for x, y in zip(work, work[1:]))
    if cus == 256:
        ws = fmha.workspace_size(p, b, 1, fmha.VARIANT_BALANCED_PAIR)
        assert ws == (m_tiles - sf) * h * b * 2 * 4 * 34 * 64 * 4



@pytest.mark.parametrize("b,h,sq,xccs,force,groups", [
    (1, 2, 40000, 8, True, 4),     # cfg5: each (batch, head) on 4 XCDs
    (1, 1, 40000, 8, True, 8),
    (1, 4, 40000, 8, True, 2),
    (1, 2, 40000, 8, "pair", 4),
    (2, 1, 60000, 8, True, 4),
    (1, 3, 40000, 8, True, 1),     # 3 does not divide 8: plain order
    (1, 2, 40000, 1, True, 1),     # one XCD: plain order
    (1, 8, 40000, 8, True, 1),     # one group: plain order
    (1, 2, 40000, 4, True, 2),     # a 4-XCD partition: 2 groups
    (1, 4, 40000, 4, True, 1),     # a 4-XCD partition, 4 heads: plain order
])
def test_balanced_plan_orders_runs_by_first_key(b, h, sq, xccs, force, groups):
    """With nhead_q * batch dividing the XCD count into groups (entry z runs
    on group z % groups), each run of `groups` consecutive entries holds the
    plain heaviest-first table's same items (so the dispatch sees the same
    work per run), ordered by the first key tile they read: whole M-tiles and
    first halves (key 0) before second halves (key ceil(n/2)), ties in the
    plain order.  Otherwise the table is the plain one."""
    p = valid_params(lse=False)
    p.nhead_q = p.nhead_k = h
    p.seqlen_q = p.seqlen_k = sq
    got, sf = fmha.balanced_plan(p, b, 1, 256, force, xccs=xccs)
    plain, sf1 = fmha.balanced_plan(p, b, 1, 256, force, xccs=1)
    assert sf == sf1 and len(got) == len(plain)
    if groups == 1:
        assert got == plain
        return
    pair = force == "pair"
    m_tiles = -(-sq // 128)

    def first_key(it):
        u, half = it
        n = _ntiles(min(2 * u + 1, m_tiles - 1) if pair else u, sq, sq)
        return (n + 1) // 2 if half == 1 else 0

    assert got != plain
    for r in range(0, len(plain), groups):
        run, want = got[r:r + groups], plain[r:r + groups]
        assert sorted(run) == sorted(want)
        assert run == sorted(want, key=lambda it: (first_key(it), want.index(it)))

@pytest.mark.parametrize("b,h,sq,causal", [(4, 16, 2048, 0), (4, 16, 2048, 1), (1, 16, 8192, 1), (1, 4, 32768, 1)])
def test_balanced_plan_only_where_the_heaviest_m_tile_outlasts_the_average(b, h, sq, causal):
    p = valid_params(lse=False)
    p.nhead_q = p.nhead_k = h
    p.seqlen_q = p.seqlen_k = sq
    assert fmha.balanced_plan(p, b, causal, 256) == ([], None)
    assert fmha.workspace_size(p, b, causal) == 0


@pytest.mark.parametrize("b,h,s,planned", [
    (1, 2, 40000, True),    # cfg5: 626 blocks, a partial second round of long M-tiles
    (1, 8, 4096, True),     # 256 blocks (one per CU), 64 key tiles
    (1, 8, 2048, True),     # 128 blocks (half a block per CU), 32 key tiles
    (1, 5, 8192, True),     # 320 blocks (1.25 per CU), 128 key tiles
    (1, 9, 8192, True),     # 576 blocks
    (1, 1, 32768, True),
    (8, 16, 256, False),    # 256 blocks of 2-4 key tiles: the merge costs more than it saves
    (16, 16, 256, False),
    (8, 16, 512, False),
    (4, 16, 1024, False),
    (1, 12, 2048, False),   # 192 blocks, 32 key tiles
    (1, 16, 2048, False),   # 256 blocks, 32 key tiles
    (1, 10, 4096, False),   # 320 blocks, 64 key tiles
    (2, 16, 2048, False),   # 512 blocks (two per CU): split-KV or regular
    (1, 16, 4096, False),
    (1, 2, 32768, False),
    (1, 20, 4096, False),   # 640 blocks, 64 key tiles
    (1, 6, 16384, False),   # 768 blocks: the heaviest M-tile is ~1.3x the average
    (1, 16, 8192, False),   # cfg3
])
def test_balanced_plan_where_it_measured_faster(b, h, s, planned):
    """The automatic choice takes a balanced plan only where the balanced form
    measured faster than the launch without a workspace (256 CUs)."""
    p = valid_params(lse=False)
    p.nhead_q = p.nhead_k = h
    p.seqlen_q = p.seqlen_k = s
    items, _ = fmha.balanced_plan(p, b, 1, 256)
    assert bool(items) == planned
    assert fmha.balanced_plan(p, b, 1, 256, True)[0]  # forced: always a plan


def test_balanced_plan_cache_follows_the_shape():
    """The launcher keeps the last plan built on a thread; alternating shapes
    (and compute-unit counts, force, causal) must each get their own plan."""
    def shape(h, s):
        p = valid_params(lse=False)
        p.nhead_q = p.nhead_k = h
        p.seqlen_q = p.seqlen_k = s
        return p

    cases = [(shape(2, 40000), 1, 256, False), (shape(1, 32768), 1, 256, False), (shape(2, 40000), 1, 128, False),
             (shape(2, 3000), 1, 256, True), (shape(2, 3000), 1, 256, False), (shape(2, 40000), 0, 256, True)]
    first = [fmha.balanced_plan(p, 1, c, cus, f) for p, c, cus, f in cases]
    assert first[0][0] and first[1][0] and first[3][0] and first[4][0]  # planned
    assert first[2] == ([], None) and first[5] == ([], None)             # 128 CUs: balanced already; not causal
    assert first[0] != first[1] and first[3] != first[0]
    for _ in range(3):
        for (p, c, cus, f), want in zip(cases, first):
            assert fmha.balanced_plan(p, 1, c, cus, f) == want


def test_ws_entry_rejects_bad_workspaces_and_forms():
    """Refused before anything is launched (no GPU needed)."""
    lib = fmha.load_library()
    p = valid_params(lse=False)
    p.nhead_q = p.nhead_k = 2
    p.seqlen_q = p.seqlen_k = 40000
    B = fmha.VARIANT_BALANCED
    need = fmha.workspace_size(p, 1, 1, B)
    assert need > 0
    ws = 1 << 20
    for args in [(1, 1, B, ws + 8, need),          # not 256-byte aligned
                 (1, 1, B, ws, need - 1),          # too small for the forced plan
                 (1, 1, B, None, 5),               # bytes without memory
                 (1, 1, B, ws, -1),
                 (1, 0, B, ws, need),              # not causal
                 (1, 1, 99, ws, need),             # unknown form
                 (1, 1, fmha.VARIANT_BALANCED_PAIR, ws, fmha.workspace_size(p, 1, 1, 7) - 1)]:
        assert lib.fmha_fwd_d64_bf16_ws(ctypes.byref(p), *args, None) == INVALID, args
    assert fmha.workspace_size(_mut(q=None), 1, 1) == -1
    assert fmha.workspace_size(p, 1, 1, fmha.VARIANT_REGULAR) == 0
    pv = valid_params(varlen=True, lse=False)      # varlen: never balanced
    assert lib.fmha_fwd_d64_bf16_ws(ctypes.byref(pv), 1, 1, B, ws, need, None) == INVALID
    assert fmha.balanced_plan(pv, 1, 1, 256, True) == ([], None)
