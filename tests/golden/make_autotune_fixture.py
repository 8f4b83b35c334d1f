"""Writes tests/golden/flexgemm_autotune_spconv.json: the three submanifold masked-implicit-GEMM sections of the
reference's FlexGEMM autotune cache (assets/flexgemm_autotune.json, device "NVIDIA H200"), the data its
spconv_cfg replays (src/spconv.cu:176-221). Run once in the build container (the GPU box has no reference):
    python tests/golden/make_autotune_fixture.py /root/reference/assets/flexgemm_autotune.json
"""
import json
import os
import sys

M = "flex_gemm.kernels.triton.spconv.sparse_submanifold_conv_fwd_masked_implicit_gemm"
SECTIONS = (M + "_splitk.sparse_submanifold_conv_fwd_masked_implicit_gemm_splitk",
            M + "_splitk.sparse_submanifold_conv_fwd_masked_implicit_gemm_splitk_kernel",
            M + ".sparse_submanifold_conv_fwd_masked_implicit_gemm_kernel")

if __name__ == "__main__":
    src = json.load(open(sys.argv[1]))
    out = {dev: {k: v for k, v in secs.items() if k in SECTIONS} for dev, secs in src.items()}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "flexgemm_autotune_spconv.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
    print(dst, sum(len(v) for d in out.values() for v in d.values()), "entries")
