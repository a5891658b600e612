"""Extract the LeNet tensors of the reference's shipped checkpoints into an npz fixture.

Reads /root/reference/examples/checkpoints/lenet5_mnist.pt (float weights) and
lenet5_mnist_static_int4.pt (packed signed INT4 codes, scales, fixed input
scales, biases, per-matrix names, seeds and read events) with
``torch.load(weights_only=True)``; the static checkpoint was produced by the
reference from the float one (examples/checkpoints/README.md:28-41), so the
pair pins weight quantization, two's complement masking, [m,p,R,C] packing,
padding and seed derivation.  The static checkpoint's whole state dict is kept
too (tensors, plus each matrix's ``_extra_state`` as JSON, and the saved
simulator Config), so that tests can load it into a converted LeNet-5 with
``load_state_dict`` as examples/04_lenet5_mnist_static_quant.py:165-185 does.
Run in the build container: python tests/golden/make_lenet_fixture.py
"""

import json

from pathlib import Path

import numpy as np
import torch

CHECKPOINTS = Path("/root/reference/examples/checkpoints")
OUT = Path(__file__).with_name("lenet_int4.npz")

# state-dict prefix of each analog matrix -> float weight name
LAYERS = {
    "features.0.matrices.0": "features.0.weight",
    "features.3.matrices.0": "features.3.weight",
    "classifier.0": "classifier.0.weight",
    "classifier.2": "classifier.2.weight",
    "classifier.4": "classifier.4.weight",
}


def main():
    digital = torch.load(CHECKPOINTS / "lenet5_mnist.pt", weights_only=True, map_location="cpu")
    static = torch.load(CHECKPOINTS / "lenet5_mnist_static_int4.pt", weights_only=True,
                        map_location="cpu")
    weights = digital["state_dict"]
    state = static["state_dict"]
    out = {}
    for index, (prefix, weight_name) in enumerate(LAYERS.items()):
        extra = state[prefix + "._extra_state"]
        out[f"l{index}_weight"] = weights[weight_name].flatten(1).numpy()
        out[f"l{index}_packed"] = state[prefix + ".packed"].numpy()
        out[f"l{index}_weight_scale"] = state[prefix + ".weight_scale"].numpy()
        out[f"l{index}_input_scale"] = state[prefix + ".input_scale"].numpy()
        out[f"l{index}_name"] = np.array(extra["name"])
        out[f"l{index}_seed"] = np.array(extra["seed"], dtype=np.uint64)
        out[f"l{index}_maximum"] = np.array(
            static["calibration"]["layers"][prefix]["maximum"], dtype=np.float64)
        out[f"l{index}_prefix"] = np.array(prefix)
        out[f"l{index}_bias"] = state[prefix + ".bias"].numpy()
        out[f"l{index}_extra_state"] = np.array(json.dumps(extra))
    out["count"] = np.array(len(LAYERS))
    out["state_keys"] = np.array(sorted(state))
    out["config"] = np.array(json.dumps(static["config"]))
    out["conversion"] = np.array(json.dumps(static["conversion"]))
    out["format"] = np.array(static["format"])
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
