"""Test problem tables.

``K_ALL_FULL`` is the reference's full-kernel matrix (``tests/test_configs.hpp:19-102``,
63 rows), kept row for row with the same names so failures map back to it.
Tuple fields follow the reference's ``TestCase``
(``tests/test_params.hpp:20-29``): name, batch, heads, seq, hdim, kv_heads,
kv_seq, mask, lse, opt, varlen_seqs; 0 means "derive" as in its
``make_params``.

``BASELINE`` are the five benchmark configurations of this build's metric.
"""
from fmha_native_amd.problem import Problem

K_ALL_FULL = [
    # === D64 Smoke ===
    ("D64Smoke1", 2, 2, 512, 64, 0, 0, 0, 0, 0),
    ("D64Smoke2", 1, 1, 256, 64, 0, 0, 0, 0, 0),
    ("D64Smoke3", 2, 4, 1024, 64, 0, 0, 0, 0, 0),
    ("D64Smoke4", 1, 8, 2048, 64, 0, 0, 0, 0, 0),
    # === D64 Feature Combos ===
    ("D64MaskLse", 2, 4, 1024, 64, 0, 0, 1, 1, 0),
    ("D64GqaMask", 2, 8, 1024, 64, 2, 0, 1, 0, 0),
    ("D64MqaMaskLse", 2, 8, 1024, 64, 1, 0, 1, 1, 0),
    ("D64AsymSqLtSkvMaskLse", 1, 8, 512, 64, 0, 1024, 1, 1, 0),
    ("D64AsymSqGtSkvMask", 1, 4, 1024, 64, 0, 512, 1, 0, 0),
    ("D64KitchenSink", 2, 8, 1024, 64, 2, 2048, 1, 1, 0),
    # === D64 Edge Cases ===
    ("D64EdgeS300MaskLse", 1, 2, 300, 64, 0, 0, 1, 1, 0),
    ("D64EdgeS300GqaMask", 1, 4, 300, 64, 2, 0, 1, 0, 0),
    ("D64EdgeS255", 1, 2, 255, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS255MaskLse", 1, 2, 255, 64, 0, 0, 1, 1, 0),
    ("D64EdgeS33MaskLse", 1, 2, 33, 64, 0, 0, 1, 1, 0),
    ("D64EdgeS33MqaMask", 1, 2, 33, 64, 1, 0, 1, 0, 0),
    ("D64EdgeS17MaskLse", 1, 1, 17, 64, 0, 0, 1, 1, 0),
    ("D64EdgeS17GqaMask", 1, 4, 17, 64, 2, 0, 1, 0, 0),
    ("D64EdgeS16", 1, 1, 16, 64, 0, 0, 0, 0, 0),
    ("D64EdgeScale", 1, 1, 8192, 64, 0, 0, 1, 1, 0),
    # === D64 Varlen ===
    ("D64VarlenMask", 4, 4, 1024, 64, 0, 0, 1, 0, 0, (512, 256, 1024, 128)),
    ("D64VarlenGqaMask", 2, 8, 512, 64, 2, 0, 1, 0, 0, (512, 256)),
    ("D64VarlenEdgeMaskLse", 2, 2, 300, 64, 0, 0, 1, 1, 0, (300, 33)),
    ("D64VarlenMqaMaskLse", 4, 8, 1024, 64, 1, 0, 1, 1, 0, (1024, 512, 256, 128)),
    # === D64 Feature Variants ===
    ("D64MaskOnly", 2, 4, 1024, 64, 0, 0, 1, 0, 0),
    ("D64LseOnly", 2, 4, 1024, 64, 0, 0, 0, 1, 0),
    ("D64GqaAsymMaskLse", 1, 8, 512, 64, 2, 1024, 1, 1, 0),
    ("D64MqaAsymMask", 1, 8, 1024, 64, 1, 512, 1, 0, 0),
    # === D64 Boundary/Misc ===
    ("D64EdgeS300", 1, 2, 300, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS256", 1, 2, 256, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS33", 1, 2, 33, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS17", 1, 1, 17, 64, 0, 0, 0, 0, 0),
    ("D64EdgeKvseq0", 1, 1, 256, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS1", 1, 1, 1, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS2Mask", 1, 2, 2, 64, 0, 0, 1, 0, 0),
    ("D64EdgeS31", 1, 2, 31, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS32", 1, 2, 32, 64, 0, 0, 1, 0, 0),
    ("D64EdgeS64MaskLse", 1, 4, 64, 64, 0, 0, 1, 1, 0),
    ("D64EdgeS257Mask", 1, 2, 257, 64, 0, 0, 1, 0, 0),
    ("D64H3Mask", 2, 3, 512, 64, 0, 0, 1, 0, 0),
    ("D64H6GqaMask", 1, 6, 1024, 64, 3, 0, 1, 0, 0),
    ("D64GqaRatio8MaskLse", 1, 16, 512, 64, 2, 0, 1, 1, 0),
    ("D64GqaNomask", 2, 8, 1024, 64, 2, 0, 0, 0, 0),
    ("D64VarlenNomask", 2, 4, 512, 64, 0, 0, 0, 0, 0, (512, 256)),
    ("D64EdgeKvseq1", 1, 2, 256, 64, 0, 1, 0, 0, 0),
    ("D64AsymLongContext", 1, 4, 64, 64, 0, 4096, 1, 1, 0),
    ("D64VarlenTinyMaskLse", 4, 2, 512, 64, 0, 0, 1, 1, 0, (1, 512, 32, 256)),
    ("D64B8Mask", 8, 4, 512, 64, 0, 0, 1, 0, 0),
    # === D64 Tile Boundary ===
    ("D64EdgeS128", 1, 2, 128, 64, 0, 0, 0, 0, 0),
    ("D64EdgeS128MaskLse", 1, 4, 128, 64, 0, 0, 1, 1, 0),
    ("D64EdgeS65MaskLse", 1, 2, 65, 64, 0, 0, 1, 1, 0),
    ("D64EdgeAsymS128Sk65Mask", 1, 2, 128, 64, 0, 65, 1, 0, 0),
    # === D64 Feature Combos (gaps) ===
    ("D64GqaLseNomask", 2, 8, 512, 64, 2, 0, 0, 1, 0),
    ("D64VarlenGqaMaskLse", 2, 8, 512, 64, 2, 0, 1, 1, 0, (512, 256)),
    ("D64VarlenLseNomask", 2, 4, 512, 64, 0, 0, 0, 1, 0, (512, 256)),
    ("D64VarlenAsymMask", 2, 4, 256, 64, 0, 512, 1, 0, 0, (256, 128)),
    # === D64 Causal full-tile-skip coverage ===
    ("D64CausalDeepSquare", 1, 2, 768, 64, 0, 0, 1, 0, 0),
    ("D64CausalDeepSquareLse", 1, 2, 768, 64, 0, 0, 1, 1, 0),
    ("D64CausalRaggedTail", 1, 2, 832, 64, 0, 0, 1, 0, 0),
    ("D64CausalDeepRagged", 1, 2, 1100, 64, 0, 0, 1, 0, 0),
    ("D64CausalShift128", 1, 2, 256, 64, 0, 384, 1, 0, 0),
    ("D64CausalShift64", 1, 2, 256, 64, 0, 320, 1, 0, 0),
    ("D64CausalGqaDeepRagged", 1, 8, 900, 64, 2, 0, 1, 0, 0),
]


def problem_from_row(row):
    name, b, h, s, d, kvh, kvs, mask, lse, _opt = row[:10]
    seqs = row[10] if len(row) > 10 else ()
    assert d == 64
    return Problem(batch=b, nhead_q=h, seqlen_q=s, nhead_k=kvh, seqlen_k=kvs, causal=bool(mask), lse=bool(lse),
                   varlen_seqs=seqs, name=name)


def all_full():
    return [problem_from_row(r) for r in K_ALL_FULL]


# Benchmark configurations (inputs N(0,1) unless noted; seed 42).
from fmha_native_amd.problem import baseline_problems  # noqa: E402,F401
