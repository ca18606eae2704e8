"""Copy the reference's real-logit greedy fixtures into tests/golden/fixtures/.

Run once in the build container (where /root/reference exists).  The copied
files are data only: the last-position fp16 logits of six real models and the
argmax the reference's mlx-lm oracle recorded for them
(reference/fixtures*/{logits_last,argmax}.npy, described in
reference/README.md; MIT licence, README.md:189).  Loaded with
numpy.load(allow_pickle=False).
"""
import os
import shutil

import numpy as np

SRC = "/root/reference/reference"
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures")
MODELS = ["fixtures", "fixtures_qwen3", "fixtures_qwen3_5", "fixtures_qwen3_moe",
          "fixtures_qwen3_vl", "fixtures_qwen3_yarn"]


def main():
    for m in MODELS:
        os.makedirs(os.path.join(DST, m), exist_ok=True)
        for f in ("logits_last.npy", "argmax.npy"):
            src = os.path.join(SRC, m, f)
            np.load(src, allow_pickle=False)  # refuse anything that is not plain data
            shutil.copyfile(src, os.path.join(DST, m, f))
    print("copied", len(MODELS), "fixture pairs to", DST)


if __name__ == "__main__":
    main()
