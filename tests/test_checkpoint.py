"""Weight files (checkpoint.py) on the CPU, with stand-in parameters: the per-layer order
and in-place semantics of the reference notebook's save_weights / load_weights (demo.ipynb
cell 17) over an .npz archive that is never unpickled."""
import json

import numpy as np
import pytest

import checkpoint


class FakeParam:
    def __init__(self, arr):
        self.a = np.array(arr, dtype=np.float32)
        self.shape = self.a.shape

    def get(self):
        return self.a.copy()

    def set(self, host):
        assert host.shape == self.shape
        self.a[...] = host


class FakeLayer:
    def __init__(self, *shapes, rng=None):
        self.parameters = [FakeParam(rng.standard_normal(s)) for s in shapes]


class Dense(FakeLayer):
    pass


class LayerNorm(FakeLayer):
    pass


class Dropout(FakeLayer):
    pass


class FakeModel:
    def __init__(self, seed, widths=(8, 16)):
        rng = np.random.default_rng(seed)
        self.layers = [Dense((widths[0], widths[1]), (widths[1],), rng=rng), Dropout(rng=rng),
                       LayerNorm((widths[1],), (widths[1],), rng=rng)]


def params(model):
    return [p.a for layer in model.layers for p in layer.parameters]


def test_round_trip_in_layer_order(tmp_path):
    a, b = FakeModel(0), FakeModel(1)
    path = str(tmp_path / "w.npz")
    checkpoint.save_weights(a, path)
    assert checkpoint.load_weights(b, path) is b
    for x, y in zip(params(a), params(b)):
        assert np.array_equal(x, y)
    with np.load(path, allow_pickle=False) as z:
        meta = json.loads(bytes(z["__layout__"]).decode())
        assert [l["name"] for l in meta["layers"]] == ["Dense", "Dropout", "LayerNorm"]
        assert sorted(k for k in z.files if k != "__layout__") == ["L0000.P00", "L0000.P01",
                                                                   "L0002.P00", "L0002.P01"]


def test_layout_mismatch_is_refused_before_any_write(tmp_path):
    path = str(tmp_path / "w.npz")
    checkpoint.save_weights(FakeModel(0), path)
    other = FakeModel(1, widths=(8, 12))
    before = [p.copy() for p in params(other)]
    with pytest.raises(ValueError, match="layer 0"):
        checkpoint.load_weights(other, path)
    for x, y in zip(before, params(other)):
        assert np.array_equal(x, y)
    short = FakeModel(1)
    short.layers = short.layers[:2]
    with pytest.raises(ValueError, match="layers"):
        checkpoint.load_weights(short, path)


def test_files_that_need_unpickling_or_lack_a_layout_are_refused(tmp_path):
    obj = str(tmp_path / "obj.npz")
    np.savez(obj, __layout__=np.array([{"format": checkpoint.FORMAT}], dtype=object))
    with pytest.raises(ValueError):
        checkpoint.load_weights(FakeModel(0), obj)
    bare = str(tmp_path / "bare.npz")
    np.savez(bare, x=np.zeros(3, np.float32))
    with pytest.raises(ValueError, match="not a"):
        checkpoint.load_weights(FakeModel(0), bare)


def test_array_mismatch_behind_a_matching_layout_is_refused_before_any_write(tmp_path):
    """The JSON layout matches the model but the last array does not: nothing is written."""
    path = str(tmp_path / "w.npz")
    checkpoint.save_weights(FakeModel(0), path)
    with np.load(path, allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    for bad in (arrays["L0002.P01"].astype(np.float64), arrays["L0002.P01"][:-1]):
        arrays["L0002.P01"] = bad
        np.savez(path, **arrays)
        other = FakeModel(1)
        before = [p.copy() for p in params(other)]
        with pytest.raises(ValueError, match="L2.P1"):
            checkpoint.load_weights(other, path)
        for x, y in zip(before, params(other)):
            assert np.array_equal(x, y)


def _notebook_save(model, path, protocol):
    """What the notebook's save_weights writes (reference demo.ipynb cell 17): a pickled
    list of {"name", "parameters"} records holding host arrays."""
    import pickle
    lst = [{"name": type(layer).__name__, "parameters": [p.get() for p in layer.parameters]}
           for layer in model.layers]
    with open(path, "wb") as f:
        pickle.dump(lst, f, protocol=protocol)


@pytest.mark.parametrize("protocol", [2, 4, 5])
def test_notebook_pickle_is_read_in_layer_order(tmp_path, protocol):
    a, b = FakeModel(0), FakeModel(1)
    path = str(tmp_path / "nb.pkl")
    _notebook_save(a, path, protocol)
    assert checkpoint.load_notebook_weights(b, path) is b
    for x, y in zip(params(a), params(b)):
        assert np.array_equal(x, y)


def test_notebook_pickle_naming_other_globals_is_refused(tmp_path):
    """A pickle that would call anything but NumPy's array reconstruction stops at the
    lookup, before the call (the payload here is a harmless print)."""
    import pickle

    class Payload:
        def __reduce__(self):
            return (print, ("called",))

    path = str(tmp_path / "evil.pkl")
    with open(path, "wb") as f:
        pickle.dump([{"name": "Dense", "parameters": [Payload()]}], f)
    with pytest.raises(pickle.UnpicklingError, match="builtins.print"):
        checkpoint.read_notebook_weights(path)
    obj = str(tmp_path / "obj.pkl")
    with open(obj, "wb") as f:
        pickle.dump([{"name": "Dense", "parameters": [np.array([1, "a"], dtype=object)]}], f)
    with pytest.raises((pickle.UnpicklingError, ValueError)):
        checkpoint.load_notebook_weights(FakeModel(0), obj)


def test_notebook_pickle_with_wrong_layout_is_refused_before_any_write(tmp_path):
    path = str(tmp_path / "nb.pkl")
    _notebook_save(FakeModel(0, widths=(8, 12)), path, 4)
    other = FakeModel(1)
    before = [p.copy() for p in params(other)]
    with pytest.raises(ValueError, match="shape"):
        checkpoint.load_notebook_weights(other, path)
    for x, y in zip(before, params(other)):
        assert np.array_equal(x, y)
