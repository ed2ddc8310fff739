"""Weight files: save_weights / load_weights for any Network of this package.

The reference notebook saves a model as a pickled list with one entry per layer,
{"name": type(layer).__name__, "parameters": [host arrays in layer.parameters order]}, and
loads it back in place, layer by layer and parameter by parameter, as float32 (reference
demo.ipynb cell 17, save_weights / load_weights). The same per-layer order and in-place
semantics are kept here, but the container is a NumPy .npz archive read with
allow_pickle=False: a pickle runs code from the file when it is loaded, an .npz holds only
arrays. Each parameter is stored as float32 under "L<layer>.P<param>" and the layout (layer
names and parameter shapes) as JSON text in "__layout__"; loading checks the layout against
the model, converts to the model's dtype (bf16 rounds to nearest even) and uploads each
parameter once. A bf16 model saved and loaded again is bit-identical.
"""
import json

import numpy as np

FORMAT = "torchless-nn-npz/1"


def _layout(model):
    return [{"name": type(layer).__name__,
             "shapes": [list(p.shape) for p in getattr(layer, "parameters", [])]}
            for layer in model.layers]


def save_weights(model, path):
    """Write every parameter of `model` (layer order, then parameter order) to `path` (.npz)."""
    arrays = {}
    for i, layer in enumerate(model.layers):
        for j, p in enumerate(getattr(layer, "parameters", [])):
            arrays[f"L{i:04d}.P{j:02d}"] = np.asarray(p.get(), dtype=np.float32)
    meta = {"format": FORMAT, "layers": _layout(model)}
    arrays["__layout__"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    with open(path, "wb") as f:
        np.savez(f, **arrays)


def load_weights(model, path):
    """Overwrite the parameters of `model` in place from a file written by save_weights.
    Raises ValueError when the file's layers or parameter shapes do not match the model."""
    with np.load(path, allow_pickle=False) as z:
        if "__layout__" not in z.files:
            raise ValueError(f"{path}: not a {FORMAT} weight file")
        meta = json.loads(bytes(z["__layout__"]).decode())
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: format {meta.get('format')!r}, expected {FORMAT!r}")
        want = _layout(model)
        if len(meta["layers"]) != len(want):
            raise ValueError(f"{path}: {len(meta['layers'])} layers, the model has {len(want)}")
        for i, (got, exp) in enumerate(zip(meta["layers"], want)):
            if got["name"] != exp["name"] or got["shapes"] != exp["shapes"]:
                raise ValueError(f"{path}: layer {i} is {got['name']} {got['shapes']}, the model "
                                 f"has {exp['name']} {exp['shapes']}")
        for i, layer in enumerate(model.layers):
            for j, p in enumerate(getattr(layer, "parameters", [])):
                arr = z[f"L{i:04d}.P{j:02d}"]
                if arr.dtype != np.float32 or list(arr.shape) != list(p.shape):
                    raise ValueError(f"{path}: L{i}.P{j} is {arr.dtype} {arr.shape}")
                p.set(arr)
    return model
