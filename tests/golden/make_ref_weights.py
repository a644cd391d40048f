"""Convert the reference's trained maze checkpoints into small weight fixtures.

Reads `runs/engine/{maze_ood_opt,maze_hard_opt}/seed0/final.pt` of the reference repository
(torch zip archives of tensors) with `torch.load(weights_only=True)`, which executes nothing from
the file, and writes the model tensors (fp32) and the model config as `ref_<name>.npz` /
`ref_<name>.json` next to this script. These are data fixtures: trained weights of the
reference's C=16 (maze_ood) and C=32 (maze_hard) cells, used to run the HIP kernels on realistic
parameters.

Usage: python tests/golden/make_ref_weights.py [/root/reference]
"""

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main(ref_root: str = "/root/reference") -> None:
    for name in ("maze_ood", "maze_hard"):
        path = os.path.join(ref_root, "runs", "engine", f"{name}_opt", "seed0", "final.pt")
        ck = torch.load(path, map_location="cpu", weights_only=True)
        tensors = {k: v.detach().to(torch.float32).numpy() for k, v in ck["model"].items()}
        np.savez_compressed(os.path.join(HERE, f"ref_{name}.npz"), **tensors)
        cfg = dict(ck["model_config"])
        cfg["output_tokens"] = list(cfg["output_tokens"])
        with open(os.path.join(HERE, f"ref_{name}.json"), "w") as f:
            json.dump(cfg, f, indent=1, sort_keys=True)
        print(name, {k: v.shape for k, v in tensors.items()})


if __name__ == "__main__":
    main(*sys.argv[1:])
