"""Runtime selector with the MI355X value (reference backend.py:1-34).

The reference picks its array module once, at import, from XP_RUNTIME (CUDA -> CuPy,
CPU -> NumPy; backend.py:3-22). This build implements one value, XP_RUNTIME=MI355X (the
default here), whose `xp` is `tl_hip`: device arrays in HBM and hand-written gfx950 kernels
behind a C ABI. CUDA and CPU are refused with an explanation rather than emulated.

FLOAT_TYPE is fp32 as in the reference (backend.py:24); XP_FLOAT=bf16 (or
set_float_type) selects bf16 storage with fp32 accumulation for layers built afterwards.
"""
import os

runtime = os.environ.get("XP_RUNTIME", "MI355X")
if runtime != "MI355X":
    raise RuntimeError(
        f"XP_RUNTIME={runtime!r} is not available in this build: it provides only the "
        "MI355X runtime (HIP kernels on a gfx950 GPU). Unset XP_RUNTIME or set it to MI355X.")

import tl_hip as xp  # noqa: E402

FLOAT_TYPE = xp.as_dtype(os.environ.get("XP_FLOAT", "fp32"))

# tensor initialization with float type (reference backend.py:27-34). The reference's
# generator is unseeded; TL_SEED seeds this one.
_seed = os.environ.get("TL_SEED")
rng = xp.random.default_rng(int(_seed) if _seed is not None else None)


def set_float_type(dtype):
    """Select fp32 or bf16 for tensors and layers created from now on."""
    global FLOAT_TYPE
    FLOAT_TYPE = xp.as_dtype(dtype)
    return FLOAT_TYPE


def init_random_tensor(size, divisor=None):
    """N(0,1) / divisor of `size` in FLOAT_TYPE, drawn on the device as the reference's
    CuPy runtime does (backend.py:27-31): a Philox draw whose key comes from the seeded
    host generator `rng`, so TL_SEED makes initialisation reproducible."""
    key = int(rng._g.integers(0, 2 ** 63))
    std = 1.0 / float(divisor) if divisor is not None else 1.0
    return xp.random_normal(tuple(size) if not isinstance(size, int) else (size,), key, 0,
                            std=std, dtype=FLOAT_TYPE)


def init_zeros_tensor(size):
    return xp.zeros(size, dtype=FLOAT_TYPE)
