"""Writes the golden fixtures of tests/golden/ (run once; the outputs are committed).

randn_seed{S}.json: torch.manual_seed(S); torch.randn(n) on the CPU, as the exact float32 bit patterns
(hex), for the sizes the reference draws with its torch_randn (engine/src/pipeline.cu:17-64): a multiple of
16 and a ragged size. torch is a third-party library here (not the reference), so running it is allowed;
it pins oracle.torch_randn.
"""
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    for seed, n in ((0, 1024), (42, 1000), (123456789, 4099)):
        torch.manual_seed(seed)
        x = torch.randn(n).numpy().astype(np.float32)
        with open(os.path.join(HERE, f"randn_seed{seed}.json"), "w") as f:
            json.dump({"seed": seed, "n": n, "torch": torch.__version__,
                       "bits": [f"{b:08x}" for b in x.view(np.uint32).tolist()]}, f)
    print("wrote randn fixtures")


if __name__ == "__main__":
    main()
