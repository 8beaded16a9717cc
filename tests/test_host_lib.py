"""The C-ABI library on the CPU: it loads, exports every declared entry
point, and its host-side formats and generator agree with the oracle and
with closed forms.  No device calls here."""
import ctypes as C
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
Q4, Q5, Q8, F32, F16 = 2, 6, 8, 0, 1


@pytest.fixture(scope="module")
def lib():
    from moe_amd import _lib

    if not _lib.LIB_PATH.exists():
        from moe_amd.build import build

        build()
    return _lib.lib()


def declared_functions():
    text = (ROOT / "include" / "moe_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_function(lib):
    names = declared_functions()
    assert len(names) >= 20
    from moe_amd import _lib

    for n in names:
        assert hasattr(lib, n), f"{n} is declared in include/moe_hip.h but not exported"
        assert n in _lib.PROTOTYPES, f"{n} has no ctypes prototype"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (moe_\w+)", out))
    assert set(names) <= exported


def test_row_bytes(lib):
    assert [lib.moe_row_bytes(dt, 4096) for dt in (F32, Q4, Q5, Q8)] == [16384, 2304, 2816, 4352]
    assert lib.moe_row_bytes(99, 32) == 0


@pytest.mark.parametrize("dt", [Q4, Q5, Q8, F16, F32])
def test_quantizer_matches_oracle(lib, oracle, dt):
    rng = np.random.default_rng(dt)
    x = (rng.standard_normal((64, 256)) * np.exp2(rng.integers(-20, 8, (64, 1)))).astype(np.float32)
    x[0, :32] = 0.0
    x[1, :32] = -0.0
    x[2, 5] = 1e-30
    x[3, :] = np.linspace(-3.5, 3.5, 256)
    mine = np.empty(64 * int(lib.moe_row_bytes(dt, 256)), dtype=np.uint8)
    assert lib.moe_quantize_rows(dt, x.ctypes.data_as(C.c_void_p), 64, 256, mine.ctypes.data_as(C.c_void_p)) == 0
    assert np.array_equal(mine, oracle.quantize(dt, x))
    back = np.empty_like(x)
    assert lib.moe_dequant_rows(dt, mine.ctypes.data_as(C.c_void_p), 64, 256, back.ctypes.data_as(C.c_void_p)) == 0
    assert np.array_equal(back.view(np.uint32), oracle.dequant(dt, mine, 64, 256).view(np.uint32))


def test_quantizer_rejects_bad_widths(lib):
    x = np.zeros((1, 48), dtype=np.float32)
    out = np.zeros(100, dtype=np.uint8)
    assert lib.moe_quantize_rows(Q4, x.ctypes.data_as(C.c_void_p), 1, 48, out.ctypes.data_as(C.c_void_p)) < 0


def _splitmix(state):
    m = (1 << 64) - 1
    z = state & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def test_splitmix64_known_answer():
    # SplitMix64 from state 0: the reference implementation's first outputs.
    g = 0x9E3779B97F4A7C15
    assert [_splitmix(g * (i + 1)) for i in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_generator_restated(lib):
    """Element 2j / 2j+1 = cos / sin half of Box-Muller pair j over splitmix64
    uniforms 2j and 2j+1 of the stream key, in double, rounded once."""
    seed, stream, n = 7, 3, 1000
    out = np.empty(n, dtype=np.float32)
    assert lib.moe_synth_normal(seed, stream, n, 0.25, 2.0, out.ctypes.data_as(C.c_void_p)) == 0
    m, g = (1 << 64) - 1, 0x9E3779B97F4A7C15
    key = _splitmix(seed) ^ _splitmix((stream * g + 1) & m)
    u = lambda i: (_splitmix((key + (i + 1) * g) & m) >> 11) * 2.0**-53
    want = []
    for j in range(n // 2):
        r = np.sqrt(-2.0 * np.log(1.0 - u(2 * j)))
        a = 6.283185307179586 * u(2 * j + 1)
        want += [0.25 + 2.0 * (r * np.cos(a)), 0.25 + 2.0 * (r * np.sin(a))]
    want = np.array(want, dtype=np.float32)
    # libm and numpy may differ in the last bit of cos/sin/log in double;
    # after rounding to float that can move a value by at most one ulp.
    assert (np.abs(out.view(np.int32) - want.view(np.int32)) <= 1).all()
    assert np.mean(out.view(np.int32) == want.view(np.int32)) > 0.999


def test_generator_statistics_and_offsets(lib):
    n = 1 << 20
    out = np.empty(n, dtype=np.float32)
    lib.moe_synth_normal(1, 9, n, 0.0, 1.0, out.ctypes.data_as(C.c_void_p))
    assert abs(out.mean()) < 5e-3 and abs(out.std() - 1) < 5e-3
    # The quantised form is the quantiser applied to the same values.
    rows, cols = 8, 128
    vals = np.empty(rows * cols, dtype=np.float32)
    lib.moe_synth_normal(3, 4, rows * cols, 0.0, 0.02, vals.ctypes.data_as(C.c_void_p))
    q = np.empty(rows * int(lib.moe_row_bytes(Q4, cols)), dtype=np.uint8)
    assert lib.moe_synth_quantized(3, 4, Q4, rows, cols, 0.0, 0.02, q.ctypes.data_as(C.c_void_p)) == 0
    ref = np.empty_like(q)
    lib.moe_quantize_rows(Q4, vals.ctypes.data_as(C.c_void_p), rows, cols, ref.ctypes.data_as(C.c_void_p))
    assert np.array_equal(q, ref)


def test_errors_without_a_device(lib):
    """With no GPU visible, context creation fails cleanly with a message."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    h = C.c_void_p()
    rc = lib.moe_ctx_create(0, C.byref(h))
    assert rc < 0 and lib.moe_last_error()


def test_bench_refuses_several_gpus():
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "8"], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 2 and "one GPU" in p.stderr
