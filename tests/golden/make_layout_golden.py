"""Writes layout_384x288_2s.json: a compact table of the expected values held by the reference's layout fixture
(engine/h3-core/tests/data/layout_384x288_2s.safetensors: the positions and table rows of a real 384x288, 2 s
pipeline call, first step). Read once with the safe loader; the committed table holds the fixture's metadata, the
segments, the table rows run-length encoded, each axis's distinct position values and their sum per segment, and
every 37th position row. The fixture comes from the PyTorch pipeline, so its float64 positions agree with the
reference's Rust layout to 1e-9 (layout.rs:278-280), not bit for bit.

    python tests/golden/make_layout_golden.py [path-to-fixture]
"""
import json
import os
import sys

import numpy as np
from safetensors import safe_open

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "/root/reference/engine/h3-core/tests/data/layout_384x288_2s.safetensors"


def main(path: str) -> None:
    with safe_open(path, "np") as f:
        meta = f.metadata()
        pos = f.get_tensor("position_ids").astype("<f8")
        rows = f.get_tensor("mod_rows").astype("<i4")
    runs = []
    for r in rows.tolist():
        if runs and runs[-1][0] == r:
            runs[-1][1] += 1
        else:
            runs.append([r, 1])
    # segment boundaries as the reference's layout test states them (layout.rs:270-277)
    segs = [(0, 137, "text"), (137, 323, "audio"), (323, 2159, "video")]
    axes = {name: [sorted(set(pos[a:b, k].tolist())) for k in range(3)] for a, b, name in segs}
    out = {
        "metadata": {k: meta[k] for k in ("text_len", "latent_t", "latent_h", "latent_w", "audio_t", "sigma")},
        "tokens": int(pos.shape[0]),
        "segments": segs,
        "mod_rows_rle": runs,
        "axis_values": axes,
        "sample_every": 37,
        "sample_rows": pos[::37].tolist(),
        "axis_sums": {name: [float(pos[a:b, k].sum()) for k in range(3)] for a, b, name in segs},
    }
    with open(os.path.join(HERE, "layout_384x288_2s.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else SRC)
