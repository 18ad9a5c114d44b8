"""Loading of the committed golden vectors (tests/golden/*.npz; written by
tests/golden/make_golden.py from the reference's own CPU renderer)."""
import glob
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RENDER_CASES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "c*.npz")))
TRAIN_CASES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "t0_*.npz")))


def load(name):
    d = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    out = {k: d[k] for k in d.files}
    for k in ("stats", "params", "cfg_json", "adam_lr_json"):
        if k in out:
            out[k] = json.loads(str(out[k]))
    for k in ("H", "W", "tile_size", "N", "sh_degree", "adam_step_in", "seed"):
        if k in out:
            out[k] = int(out[k])
    return out
