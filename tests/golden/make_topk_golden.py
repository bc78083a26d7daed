"""Write tests/golden/topk_golden.npz from the reference's torch_fused_topk.

Routing is the one function of the path that no closed form pins completely:
which of several exactly tied experts torch.topk returns, and the exact fp32
bits of torch.softmax, are properties of the reference's torch call. This
script runs that call (reframework/moe/fused.py:32-46) on fixed inputs and
stores inputs and outputs as a fixture; the tests never import the reference.

Development host only (the reference tree is not present where the GPU tests run):

    python tests/golden/make_topk_golden.py

Bytecode shipped inside the reference tree is never loaded: the script points
sys.pycache_prefix at a scratch directory before importing, so the modules are
compiled from their source files.
"""

from __future__ import annotations

import os
import sys
import tempfile

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))


def main() -> None:
    sys.pycache_prefix = tempfile.mkdtemp(prefix="ref_pycache_")
    sys.dont_write_bytecode = True
    sys.path.insert(0, REF)
    sys.path.insert(0, REPO)
    from reframework.moe.fused import torch_fused_topk  # noqa: E402  (reference)
    from reframework_amd.synth import normal  # noqa: E402

    cases = {}

    def add(name: str, logits: np.ndarray, k: int, renorm: bool) -> None:
        lg = torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32))
        w, ids = torch_fused_topk(lg, k, renorm)
        cases[f"{name}__logits"] = lg.numpy()
        cases[f"{name}__k"] = np.array(k)
        cases[f"{name}__renorm"] = np.array(int(renorm))
        cases[f"{name}__w"] = w.numpy()
        cases[f"{name}__ids"] = ids.numpy().astype(np.int64)

    # continuous fp32 logits: exact ties have probability ~0
    add("rand_e8_k2", normal(512 * 8, 10).reshape(512, 8), 2, True)
    add("rand_e8_k2_norenorm", normal(512 * 8, 11).reshape(512, 8), 2, False)
    add("rand_e16_k2", normal(512 * 16, 12).reshape(512, 16), 2, True)
    add("rand_e64_k6", normal(512 * 64, 13).reshape(512, 64), 6, True)
    add("rand_e8_k1", normal(256 * 8, 14).reshape(256, 8), 1, True)
    add("rand_e8_k8", normal(256 * 8, 15).reshape(256, 8), 8, False)
    add("rand_e256_k8", normal(64 * 256, 16).reshape(64, 256), 8, True)
    # bf16-rounded logits, as a bf16 model's F.linear produces: frequent ties
    bf = torch.from_numpy(normal(1024 * 8, 17, sigma=1.3).reshape(1024, 8)).to(torch.bfloat16)
    add("bf16_e8_k2", bf.float().numpy(), 2, True)
    bf64 = torch.from_numpy(normal(512 * 64, 18, sigma=1.3).reshape(512, 64)).to(torch.bfloat16)
    add("bf16_e64_k6", bf64.float().numpy(), 6, True)
    # constructed ties
    tie = np.array([
        [0, 0, 0, 0, 0, 0, 0, 0],
        [1, 2, 2, 1, 2, 0, 0, 0],
        [5, 5, 1, 1, 1, 1, 1, 1],
        [3, 1, 3, 2, 0, 0, 0, 0],
        [0, 5, 5, 5, 1, 5, 0, 0],
        [-1, -1, -1, 4, -1, -1, 4, -1],
        [2, 1, 0, -1, -2, -3, -4, -5],
        [-5, -4, -3, -2, -1, 0, 1, 2],
    ], dtype=np.float32)
    add("ties_e8_k2", tie, 2, True)
    add("ties_e8_k3", tie, 3, True)

    out = os.path.join(HERE, "topk_golden.npz")
    np.savez_compressed(out, **cases)
    print(f"wrote {out}: {len(cases) // 5} cases, torch {torch.__version__}")


if __name__ == "__main__":
    main()
