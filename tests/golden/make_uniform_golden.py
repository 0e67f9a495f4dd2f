"""Write the golden vectors for uniform per-channel keys.

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_uniform_golden.py /path/to/reference

The reference's uniform asymmetric per-channel key quantizer
(``PerChannelKV(bits=4)`` without NF4: turboquant_pro/per_channel_kv.py:303-317
and its decompress, :529-530) is pinned by no committed array, so this
script runs it on seeded fp16-valued inputs -- a 256-token group and an odd
200-token one, 2 % fp16 outliers -- and stores inputs and outputs only.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def main(ref: str) -> None:
    sys.path.insert(0, ref)
    from turboquant_pro.per_channel_kv import PerChannelKV

    out = {}
    for tag, S, seed in (("s256", 256, 31), ("s200", 200, 32)):
        rng = np.random.default_rng(seed)
        H, D = 2, 128
        scale = rng.lognormal(0.0, 1.0, size=(H, 1, D)).astype(np.float32)
        x = (rng.standard_normal((H, S, D)).astype(np.float32) * scale
             + rng.uniform(-1, 1, size=(H, 1, D)).astype(np.float32))
        x = x.astype(np.float16).astype(np.float32)[None]
        pk = PerChannelKV(head_dim=D, n_heads=H, bits=4, outlier_frac=0.02)
        c = pk.compress(x, packed=True)
        out[f"{tag}_x"] = x[0]
        out[f"{tag}_kpacked"] = c.indices
        out[f"{tag}_scale"] = c.scale[0, :, 0, :]
        out[f"{tag}_zero"] = c.zero[0, :, 0, :]
        out[f"{tag}_oidx"] = c.outlier_idx
        out[f"{tag}_oval"] = c.outlier_val
        out[f"{tag}_decompressed"] = pk.decompress(c)[0]
    np.savez_compressed(HERE / "perchannel_uniform.npz", **out)
    print("done")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
