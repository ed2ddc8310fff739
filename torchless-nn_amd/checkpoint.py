"""Weight files: save_weights / load_weights for any Network of this package, and a
weights-only reader for the notebook's own pickle files.

The reference notebook saves a model as a pickled list with one entry per layer,
{"name": type(layer).__name__, "parameters": [host arrays in layer.parameters order]}, and
loads it back in place, layer by layer and parameter by parameter, as float32 (reference
demo.ipynb cell 17, save_weights / load_weights). The same per-layer order and in-place
semantics are kept here, but the container is a NumPy .npz archive read with
allow_pickle=False: a pickle runs code from the file when it is loaded, an .npz holds only
arrays. Each parameter is stored as float32 under "L<layer>.P<param>" and the layout (layer
names and parameter shapes) as JSON text in "__layout__"; loading checks the layout and every
array's dtype and shape against the model before any parameter is written, converts to the
model's dtype (bf16 rounds to nearest even) and uploads each parameter once. A bf16 model
saved and loaded again is bit-identical.

load_notebook_weights reads a file the notebook's save_weights wrote. Its unpickler resolves
only NumPy's array-reconstruction callables (ndarray, dtype, _reconstruct, _frombuffer); any
other global in the file (a function, a class, a module attribute) stops the load with
pickle.UnpicklingError before it is called, so the file can only describe arrays, lists,
dicts and strings (protocol-2 files also spell bytes as a latin-1 text conversion, which is
performed by a local function that does nothing else).
"""
import io
import json
import pickle

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


def _write_checked(model, entries, where):
    """entries[i] = (layer name, [arrays]) for model.layers[i]. Checks every layer name and
    every array's shape (and that it is real-valued) first; only then uploads, so a mismatch
    leaves the model untouched."""
    layers = model.layers
    if len(entries) != len(layers):
        raise ValueError(f"{where}: {len(entries)} layers, the model has {len(layers)}")
    plan = []
    for i, (layer, (name, arrays)) in enumerate(zip(layers, entries)):
        params = getattr(layer, "parameters", [])
        if name != type(layer).__name__:
            raise ValueError(f"{where}: layer {i} is {name}, the model has {type(layer).__name__}")
        if len(arrays) != len(params):
            raise ValueError(f"{where}: layer {i} ({name}) has {len(arrays)} parameters, the "
                             f"model has {len(params)}")
        for j, (p, a) in enumerate(zip(params, arrays)):
            if not isinstance(a, np.ndarray) or a.dtype.kind not in "fiu":
                raise ValueError(f"{where}: L{i}.P{j} is not a real-valued array")
            if tuple(a.shape) != tuple(p.shape):
                raise ValueError(f"{where}: L{i}.P{j} has shape {a.shape}, the model {p.shape}")
            plan.append((p, a))
    for p, a in plan:
        p.set(np.asarray(a, dtype=np.float32))
    return model


def load_weights(model, path):
    """Overwrite the parameters of `model` in place from a file written by save_weights.
    Raises ValueError, with no parameter written, when the file's layers, parameter shapes or
    dtypes do not match the model."""
    with np.load(path, allow_pickle=False) as z:
        if "__layout__" not in z.files:
            raise ValueError(f"{path}: not a {FORMAT} weight file")
        meta = json.loads(bytes(z["__layout__"]).decode())
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: format {meta.get('format')!r}, expected {FORMAT!r}")
        want = _layout(model)
        if len(meta["layers"]) != len(want):
            raise ValueError(f"{path}: {len(meta['layers'])} layers, the model has {len(want)}")
        entries = []
        for i, (got, exp) in enumerate(zip(meta["layers"], want)):
            if got["name"] != exp["name"] or got["shapes"] != exp["shapes"]:
                raise ValueError(f"{path}: layer {i} is {got['name']} {got['shapes']}, the model "
                                 f"has {exp['name']} {exp['shapes']}")
            arrays = []
            for j in range(len(exp["shapes"])):
                arr = z[f"L{i:04d}.P{j:02d}"]
                if arr.dtype != np.float32:
                    raise ValueError(f"{path}: L{i}.P{j} is {arr.dtype}, expected float32")
                arrays.append(arr)
            entries.append((got["name"], arrays))
    return _write_checked(model, entries, path)


# globals a pickled NumPy array may name, under NumPy 1.x and 2.x module paths
_ARRAY_GLOBALS = {
    ("numpy", "ndarray"), ("numpy", "dtype"),
    ("numpy.core.multiarray", "_reconstruct"), ("numpy._core.multiarray", "_reconstruct"),
    ("numpy.core.numeric", "_frombuffer"), ("numpy._core.numeric", "_frombuffer"),
}


def _latin1_bytes(text, encoding="latin1", errors="strict"):
    """Protocol-2 pickles spell a bytes object as _codecs.encode(text, "latin1"); only that
    conversion is performed."""
    if not isinstance(text, str) or encoding not in ("latin1", "latin-1"):
        raise pickle.UnpicklingError("weight file asks for a text encoding other than latin-1")
    return text.encode("latin1")


class _ArrayOnlyUnpickler(pickle.Unpickler):
    def find_class(self, module, name):
        if (module, name) in _ARRAY_GLOBALS:
            return super().find_class(module, name)
        if (module, name) == ("_codecs", "encode"):
            return _latin1_bytes
        raise pickle.UnpicklingError(f"weight file names {module}.{name}; only NumPy arrays are "
                                     f"accepted")


def read_notebook_weights(path):
    """The [(layer name, [arrays])] list of a file written by the notebook's save_weights
    (reference demo.ipynb cell 17), read without resolving anything but NumPy's array
    reconstruction."""
    with open(path, "rb") as f:
        data = f.read()
    lst = _ArrayOnlyUnpickler(io.BytesIO(data)).load()
    if not isinstance(lst, list):
        raise ValueError(f"{path}: expected a list of layers, found {type(lst).__name__}")
    out = []
    for i, d in enumerate(lst):
        if not (isinstance(d, dict) and isinstance(d.get("name"), str)
                and isinstance(d.get("parameters"), list)):
            raise ValueError(f"{path}: entry {i} is not a {{'name', 'parameters'}} layer record")
        out.append((d["name"], d["parameters"]))
    return out


def load_notebook_weights(model, path):
    """The notebook's load_weights (reference demo.ipynb cell 17): every parameter of every
    layer overwritten in place, in order, converted to float32 (then to the model's dtype).
    Unlike the notebook's zip(), a file whose layers or shapes differ from the model is
    refused, with nothing written."""
    return _write_checked(model, read_notebook_weights(path), path)
