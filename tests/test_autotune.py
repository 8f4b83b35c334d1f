"""spconv_cfg_autotune (host only): the reference's tile choice replayed from a FlexGEMM autotune cache file
(src/spconv.cu:176-221), on the cache's submanifold sections (tests/golden/flexgemm_autotune_spconv.json, written by
tests/golden/make_autotune_fixture.py from the reference's assets/flexgemm_autotune.json)."""
import json
import os
import re

import pytest

import spconv_amd as sp

FIX = os.path.join(os.path.dirname(__file__), "golden", "flexgemm_autotune_spconv.json")
DEV = "NVIDIA H200"
M = "flex_gemm.kernels.triton.spconv.sparse_submanifold_conv_fwd_masked_implicit_gemm"


@pytest.mark.parametrize("N,Ci,Co,expect", [
    (1 << 18, 128, 128, (64, 32, 1)),        # main kernel table, non-default tile
    ((1 << 18) - 1, 128, 128, None),         # one row fewer: log2 bucket 17
    (1 << 10, 1024, 1024, (128, 64, 8)),     # split 8: the split-K kernel's entry, not the main table's (32, 32)
    ((1 << 11) - 1, 1024, 1024, (128, 64, 8)),
    (1 << 20, 64, 64, (128, 32, 1)),
    (1 << 16, 128, 128, (64, 32, 1)),
    (1000, 48, 48, (128, 64, 1)),            # no entry: the fallback
])
def test_known_answers(N, Ci, Co, expect):
    got = sp.spconv_cfg_autotune(FIX, DEV, N, Ci, Co)
    if expect is None:
        expect = reference_walk(json.load(open(FIX)), N, Ci, Co)
    assert got == expect


def reference_walk(doc, N, Ci, Co):
    """The replay rule on the parsed JSON: S from "(2^L, Ci, Co, 27)", then (B1, BK) from the split-K kernel
    section (keys with S) overridden by the main kernel section (keys without S, S = 1)."""
    d = doc.get(DEV, {})
    L = max(N, 1).bit_length() - 1
    S = d.get(M + "_splitk.sparse_submanifold_conv_fwd_masked_implicit_gemm_splitk", {}).get(
        f"(2^{L}, {Ci}, {Co}, 27)", {}).get("SPLITK", 1)
    tiles = {}
    for sec in (M + "_splitk.sparse_submanifold_conv_fwd_masked_implicit_gemm_splitk_kernel",
                M + ".sparse_submanifold_conv_fwd_masked_implicit_gemm_kernel"):
        for k, v in d.get(sec, {}).items():
            m = re.match(r"\((\d+), (\d+), (\d+), 27, (?:(\d+), )?True", k)
            if m:
                tiles[(int(m[1]), int(m[2]), int(m[3]), int(m[4] or 1))] = (v["kwargs"]["B1"], v["kwargs"]["BK"])
    return tiles.get((L, Ci, Co, S), (128, 64)) + (S,)


def test_every_entry():
    doc = json.load(open(FIX))
    shapes = set()
    for sec in doc[DEV].values():
        for k in sec:
            nums = re.findall(r"\d+", k.replace("2^", ""))
            shapes.add((int(nums[0]), int(nums[1]), int(nums[2])))
    assert len(shapes) > 20
    for L, Ci, Co in sorted(shapes):
        for N in (1 << L, (2 << L) - 1):
            assert sp.spconv_cfg_autotune(FIX, DEV, N, Ci, Co) == reference_walk(doc, N, Ci, Co), (N, Ci, Co)


def test_unknown_device_and_missing_file():
    assert sp.spconv_cfg_autotune(FIX, "AMD Instinct MI355X", 1 << 18, 128, 128) == (128, 64, 1)
    with pytest.raises(RuntimeError):
        sp.spconv_cfg_autotune(FIX + ".missing", DEV, 100, 64, 64)


def test_strict_replay(monkeypatch):
    """Strict replay (src/spconv.cu:219): a hit returns the replayed tile, a miss is an error instead of the default,
    by argument or by T2_STRICT=1 in the environment (which the plain entry point honours too)."""
    assert sp.spconv_cfg_autotune(FIX, DEV, 1 << 18, 128, 128, strict=True) == (64, 32, 1)
    with pytest.raises(RuntimeError, match="no autotune entry"):
        sp.spconv_cfg_autotune(FIX, DEV, 1000, 48, 48, strict=True)
    with pytest.raises(RuntimeError, match="no autotune entry"):
        sp.spconv_cfg_autotune(FIX, "AMD Instinct MI355X", 1 << 18, 128, 128, strict=True)
    assert sp.spconv_cfg_autotune(FIX, DEV, 1000, 48, 48) == (128, 64, 1)
    monkeypatch.setenv("T2_STRICT", "1")
    with pytest.raises(RuntimeError, match="no autotune entry"):
        sp.spconv_cfg_autotune(FIX, DEV, 1000, 48, 48)
    monkeypatch.setenv("T2_STRICT", "0")
    assert sp.spconv_cfg_autotune(FIX, DEV, 1000, 48, 48) == (128, 64, 1)
