"""CPU checks of the C-ABI boundary and the host logic (no kernel is launched here)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "libtl.h")
PKG = os.path.join(ROOT, "torchless-nn_amd")
LIB = os.path.join(PKG, "libtl.so")

needs_lib = pytest.mark.skipif(not os.path.exists(LIB), reason="libtl.so not built")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_table():
    import tl_hip
    assert header_functions() == sorted(tl_hip.SIGNATURES)


def _ctype_of(decl):
    """C parameter declaration -> the ctypes type the binding must use."""
    import ctypes as C
    decl = re.sub(r"\bconst\b", "", decl).strip()
    if "*" in decl:
        base = decl.split("*")[0].strip()
        stars = decl.count("*")
        scalar = {"int": C.c_int, "int64_t": C.c_int64, "size_t": C.c_size_t,
                  "float": C.c_float, "double": C.c_double}
        if stars == 1 and base in scalar:
            return ("ptr", scalar[base])
        return ("ptr", None)
    base = decl.rsplit(" ", 1)[0].strip()
    return {"int": C.c_int, "int32_t": C.c_int32, "int64_t": C.c_int64, "uint32_t": C.c_uint32,
            "uint64_t": C.c_uint64, "size_t": C.c_size_t, "float": C.c_float,
            "double": C.c_double}[base]


def test_binding_argument_types_match_the_header():
    """Every prototype's parameter types, position by position, against SIGNATURES."""
    import ctypes as C
    import tl_hip
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    protos = re.findall(r"\b(?:int|const char\*)\s+(tl_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text)
    assert sorted(n for n, _ in protos) == sorted(tl_hip.SIGNATURES)
    for name, params in protos:
        params = params.strip()
        decls = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        got = tl_hip.SIGNATURES[name]
        assert len(decls) == len(got), name
        for i, (d, t) in enumerate(zip(decls, got)):
            want = _ctype_of(d)
            if isinstance(want, tuple):
                if want[1] is None:
                    assert t is C.c_void_p or issubclass(t, C._Pointer), (name, i, d)
                else:
                    assert t is C.c_void_p or t == C.POINTER(want[1]), (name, i, d)
            else:
                assert C.sizeof(t) == C.sizeof(want) and (t in (C.c_float, C.c_double)) == \
                    (want in (C.c_float, C.c_double)), (name, i, d, t, want)


@needs_lib
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [f for f in header_functions() if not hasattr(lib, f)]
    assert not missing, missing


@needs_lib
def test_exported_symbols_are_exactly_the_header():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r" T (tl_[a-z0-9_]+)$", out, flags=re.M)))
    assert exported == header_functions()


def test_gemm_desc_layout_matches_header():
    """The ctypes struct must mirror tl_gemm_desc field for field."""
    import tl_hip
    text = open(HEADER).read()
    body = re.search(r"typedef struct tl_gemm_desc \{(.*?)\} tl_gemm_desc;", text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        decl = re.sub(r"^(const\s+)?(void\s*\*|double\s*\*|float\s*\*|int64_t|int32_t|float)\s*",
                      "", decl)
        names += [re.sub(r"[\s*]", "", n) for n in decl.split(",")]
    assert names == [f[0] for f in tl_hip._GemmDesc._fields_]


@needs_lib
def test_no_device_is_a_clean_error():
    """This container has no GPU: tl_init must fail with TL_ERR_NO_DEVICE and a message,
    and the Python runtime must raise rather than fall back to the CPU."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import tl_hip\n"
        "try:\n"
        "    tl_hip.ctx()\n"
        "except tl_hip.NoDeviceError as e:\n"
        "    print('NODEV', e)\n"
        "else:\n"
        "    print('HAVE_DEVICE')\n" % PKG)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    if "HAVE_DEVICE" in r.stdout:
        pytest.skip("a GPU is present")
    assert "NODEV" in r.stdout, r.stdout + r.stderr
    assert "device" in r.stdout.lower()


@needs_lib
def test_null_arguments_are_rejected_without_a_context():
    lib = ctypes.CDLL(LIB)
    lib.tl_init.argtypes = [ctypes.c_int, ctypes.c_void_p]
    lib.tl_last_error.restype = ctypes.c_char_p
    assert lib.tl_init(0, None) == 1  # TL_ERR_INVALID
    assert b"null" in lib.tl_last_error()
    lib.tl_sync.argtypes = [ctypes.c_void_p]
    assert lib.tl_sync(None) == 1


def test_missing_library_fails_loudly(tmp_path):
    code = (
        "import os, sys; os.environ['TL_LIBRARY'] = %r; sys.path.insert(0, %r)\n"
        "import tl_hip\n"
        "try:\n"
        "    tl_hip.load_library()\n"
        "except ImportError as e:\n"
        "    print('IMPORTERROR', e)\n" % (str(tmp_path / "nope.so"), PKG))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "IMPORTERROR" in r.stdout, r.stdout + r.stderr


def test_other_runtimes_are_refused():
    for value in ("CUDA", "CPU"):
        code = "import os, sys; os.environ['XP_RUNTIME'] = %r; sys.path.insert(0, %r)\nimport backend\n" % (value, PKG)
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
        assert r.returncode != 0 and "MI355X" in r.stderr


def test_host_bf16_conversion_matches_oracle():
    import tl_hip
    from oracle import numpy_ref as ref
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 100
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    assert np.array_equal(tl_hip.f32_to_bf16_bits(x), ref.bf16_bits(x))
    bits = tl_hip.f32_to_bf16_bits(x)
    assert np.array_equal(tl_hip.bf16_bits_to_f32(bits), ref.from_bf16_bits(bits))


def test_dtype_mapping():
    import tl_hip
    assert tl_hip.as_dtype(np.float64) is tl_hip.float32
    assert tl_hip.as_dtype(np.uint8) is tl_hip.uint8
    assert tl_hip.as_dtype(np.int64) is tl_hip.int64
    assert tl_hip.as_dtype(np.int16) is tl_hip.int32
    assert tl_hip.as_dtype("bf16") is tl_hip.bfloat16
    with pytest.raises(TypeError):
        tl_hip.as_dtype(np.complex64)


SAN_LIB = os.path.join(PKG, "csrc", "_build", "san", "libtl_san.so")


def _asan_runtime():
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-print-file-name=libclang_rt.asan-x86_64.so"],
                       capture_output=True, text=True)
    path = r.stdout.strip()
    return path if r.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


def test_abi_host_paths_under_address_and_ub_sanitizers():
    """Every exported entry point, called the way a binding could get it wrong (null context,
    null pointers, zero sizes) and through the no-device path, in a host build instrumented
    with ASan and UBSan: each returns a status with a message and no sanitizer reports."""
    # incremental: rebuilt when a source or header is newer than the instrumented library
    r = subprocess.run(["make", "-C", os.path.join(PKG, "csrc"), "san", "-j8"],
                       capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        pytest.skip("sanitizer build unavailable: " + r.stderr[-500:])
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("clang ASan runtime not found")
    code = (
        "import ctypes, sys; sys.path.insert(0, %r)\n"
        "import tl_hip\n"
        "lib = tl_hip.load_library()\n"
        "assert lib.tl_version() >= 1\n"
        "n = ctypes.c_int(-1)\n"
        "rc = lib.tl_device_count(ctypes.byref(n)); print('count', rc, n.value)\n"
        "h = ctypes.c_void_p()\n"
        "rc = lib.tl_init(0, ctypes.byref(h)); print('init', rc, lib.tl_last_error())\n"
        "assert rc != 0 and lib.tl_last_error()\n"
        "for name, argtypes in tl_hip.SIGNATURES.items():\n"
        "    if name in ('tl_version', 'tl_last_error'):\n"
        "        continue\n"
        "    args = []\n"
        "    for t in argtypes:\n"
        "        if t is ctypes.c_void_p or hasattr(t, '_type_') and not isinstance(t._type_, str):\n"
        "            args.append(None)\n"
        "        elif t in (ctypes.c_float, ctypes.c_double):\n"
        "            args.append(0.0)\n"
        "        else:\n"
        "            args.append(0)\n"
        "    rc = getattr(lib, name)(*args)\n"
        "    assert 0 <= rc <= 6, (name, rc)\n"
        "    if name != 'tl_event_destroy':\n"
        "        assert rc != 0 and lib.tl_last_error(), name\n"
        "print('SAN_OK')\n" % PKG)
    env = dict(os.environ, TL_LIBRARY=SAN_LIB, LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                       env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "SAN_OK" in r.stdout, out[-3000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-3000:]
