"""The committed golden fixtures (tests/golden/, written by make_golden.py
from the C oracle) against the oracle as it is now: the files are the ones
the manifest names, the seeded generator still builds the same GGUF images,
and the oracle still produces the stored logits, indices, weights, outputs
and dequantised rows bit for bit.  CPU only; the GPU tests compare the HIP
path against the same fixtures."""
import hashlib
import json
import os

import numpy as np
import pytest

import orome_amd
import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))
CASES = sorted(n[:-4] for n in MANIFEST if n != "full_rows.npz")


def load(name):
    path = os.path.join(GOLDEN, name + ".npz")
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == MANIFEST[name + ".npz"], name
    return np.load(path)


def case_model(f):
    kw = json.loads(str(f["spec"]))
    img = orome_amd.synth_gguf(orome_amd.make_spec(**kw))
    assert hashlib.sha256(img.tobytes()).hexdigest() == str(f["image_sha256"]), "generator changed"
    return img


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden_case(name):
    f = load(name)
    img = case_model(f)
    om = O.OracleModel(img)
    out, dbg = om.forward(0, f["x"], f["h"], K=int(f["K"]), omp=False, debug=True)
    for k in ("logits", "idx", "w"):
        assert np.array_equal(dbg[k].view(np.uint32), f[k].view(np.uint32)), k
    assert np.array_equal(out.view(np.uint32), f["out"].view(np.uint32))
    # and the fixture is not degenerate: outputs moved away from the residual
    assert np.linalg.norm(f["out"] - f["h"]) > 1e-3 * np.linalg.norm(f["h"])


def test_oracle_reproduces_golden_rows():
    f = load("full_rows")
    for fmt, typ, width in (("Q4_K", O.Q4_K, 2048), ("Q5_K", O.Q5_K, 512), ("Q6_K", O.Q6_K, 512),
                            ("Q8_0", O.Q8_0, 512)):
        blocks, values = f[fmt + "_blocks"], f[fmt + "_values"]
        got = O.decode_rows(typ, blocks, values.shape[0], width)
        assert np.array_equal(got.view(np.uint32), values.view(np.uint32)), fmt
