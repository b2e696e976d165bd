"""Writes the golden fixtures of the MoE path from the C oracle.

Run from the repository root:  python tests/golden/make_golden.py
It rewrites tests/golden/*.npz and tests/golden/manifest.json.

Each fixture is data only: the synthetic model's spec (the seeded generator
re-creates the GGUF image; its SHA-256 is stored so a change to the generator
shows), the seeded inputs and the oracle's outputs (router logits, expert
indices, routing weights, h_out), plus one set of full-size dequantised rows
per quant format.  tests/test_golden.py checks that the oracle still
reproduces them bit for bit and the GPU tests compare the HIP path against
them, so a coordinated change of the oracle and a kernel cannot go unnoticed.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import orome_amd  # noqa: E402
import oracle as O  # noqa: E402

# name -> (spec keyword arguments, T, K or None, input seed)
CASES = {
    "mini_q4k": (dict(layers=1, H=512, E=16, K=4, M=256, S=256, seed=101), 4, None, 11),
    "mini_q6k_down_zipf": (dict(layers=1, H=512, E=16, K=4, M=256, S=256, down=14, zipf=True, seed=102), 5, None, 12),
    "mini_q5k_down_q8_shared": (dict(layers=1, H=512, E=16, K=4, M=256, S=256, down=13, shared=8, seed=103), 3,
                                None, 13),
    "mini_no_shared_k8": (dict(layers=1, H=512, E=16, K=8, M=256, S=0, seed=104), 6, None, 14),
    "config0_b1": (dict(layers=1, H=2048, E=256, K=8, M=512, S=512, seed=105), 1, None, 15),
}
# full-size row sets: (format name, ggml type, tensor, rows, width)
ROWS = [("Q4_K", 12, "blk.0.ffn_gate_exps.weight", 4, 2048),
        ("Q5_K", 13, "blk.0.ffn_down_exps.weight", 4, 512),
        ("Q6_K", 14, "blk.0.ffn_down_exps.weight", 4, 512),
        ("Q8_0", 8, "blk.0.ffn_down_shexp.weight", 4, 512)]


def sha(b):
    return hashlib.sha256(np.ascontiguousarray(b).tobytes()).hexdigest()


def spec_of(kw):
    return orome_amd.make_spec(**kw)


def case_inputs(H, T, seed):
    x = orome_amd.synth_normal(seed, 1, T * H).reshape(T, H)
    h = orome_amd.synth_normal(seed, 2, T * H).reshape(T, H)
    return x, h


def main():
    manifest = {}
    for name, (kw, T, K, seed) in CASES.items():
        img = orome_amd.synth_gguf(spec_of(kw))
        om = O.OracleModel(img)
        x, h = case_inputs(om.H, T, seed)
        out, dbg = om.forward(0, x, h, K=K, omp=False, debug=True)
        path = os.path.join(HERE, name + ".npz")
        np.savez(path, spec=json.dumps(kw), T=T, K=K if K else om.K, image_sha256=sha(img), x=x, h=h,
                 logits=dbg["logits"], idx=dbg["idx"], w=dbg["w"], out=out)
        manifest[name + ".npz"] = hashlib.sha256(open(path, "rb").read()).hexdigest()
    rows = {}
    for fmt, typ, tensor, n, width in ROWS:
        kw = dict(layers=1, H=2048, E=8, K=2, M=512, S=512, seed=106,
                  down=typ if tensor.startswith("blk.0.ffn_down_exps") else 12,
                  shared=typ if "shexp" in tensor else 12)
        img = orome_amd.synth_gguf(spec_of(kw))
        om = O.OracleModel(img)
        dims, t, off, nb = om.tensors[tensor]
        assert t == typ, (fmt, t)
        rb = {12: 144, 13: 176, 14: 210, 8: 34}[typ] * width // (256 if typ != 8 else 32)
        blocks = img[off:off + n * rb].copy()
        rows[fmt + "_blocks"] = blocks
        rows[fmt + "_values"] = O.decode_rows(O.GGML_TO_FMT[typ], blocks, n, width)
    path = os.path.join(HERE, "full_rows.npz")
    np.savez(path, **rows)
    manifest["full_rows.npz"] = hashlib.sha256(open(path, "rb").read()).hexdigest()
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", len(manifest), "fixtures")


if __name__ == "__main__":
    main()
