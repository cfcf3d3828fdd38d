"""Temperature sampling on the CPU: the pieces the device sampler is checked against.

* sapphire_amd/csrc/libm_expf.h (the device's expf) compiled for the host agrees with this
  host's glibc expf on every float in [-104, 0], the range sample_temperature feeds it.
* The oracle's draw (oracle_sample: vec_scale by 1/T, then sample_temperature) agrees with the
  compiled reference's vec_scale + sample_temperature (utils.c:87-92, 158-180) on the token
  and on the weights left in the row, with r taken from the same libc rand() stream the
  reference draws from (srand(seed) before each).
* Hand cases fixed by the definition: r = 0, r = 1, one logit, NaN / inf rows, and draws equal
  to a running-sum value.
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from oracle.oracle import Reference

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBC = C.CDLL("libc.so.6")
LIBC.rand.restype = C.c_int
LIBC.srand.argtypes = [C.c_uint]
RAND_MAX = 2147483647

_EXPF_PROBE = r"""
#include "libm_expf.h"
#include <cmath>
#include <cstdio>
int main() {
    long bad = 0, n = 0;
#pragma omp parallel for reduction(+ : bad, n) schedule(static)
    for (long u = 0x80000000L; u <= 0xC2D00000L; ++u) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        const float a = expf(x), c = sapphire::libm_expf(x);
        if (memcmp(&a, &c, 4)) ++bad;
        ++n;
    }
    const float sp[] = {-INFINITY, INFINITY, NAN, 88.5f, 89.0f, -103.9f, -104.5f, 1.0f, 0.5f, 10.0f, 0x1p-30f};
    for (float x : sp) {
        const float a = expf(x), c = sapphire::libm_expf(x);
        if (!(a == c || (a != a && c != c))) ++bad;
    }
    printf("%ld %ld\n", n, bad);
    return 0;
}
"""


def test_libm_expf_matches_glibc_on_every_input(tmp_path):
    src = tmp_path / "probe.cpp"
    src.write_text(_EXPF_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["g++", "-O2", "-fopenmp", "-I", os.path.join(ROOT, "sapphire_amd", "csrc"), str(src), "-o",
                    str(exe), "-lm"], check=True)
    n, bad = map(int, subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split())
    assert n == 0xC2D00000 - 0x80000000 + 1
    assert bad == 0


def _rows(n, seed):
    """Logit rows of several shapes: flat, peaked, very wide, ties, special values."""
    g = np.random.default_rng(seed)
    rows = {
        "normal1": g.standard_normal(n).astype(np.float32),
        "normal4": (g.standard_normal(n) * 4).astype(np.float32),
        "wide60": (g.standard_normal(n) * 60).astype(np.float32),
        "equal": np.full(n, 0.25, np.float32),
    }
    if n >= 8:
        r = g.standard_normal(n).astype(np.float32)
        r[3] = np.nan
        rows["nan_mid"] = r
        r = g.standard_normal(n).astype(np.float32)
        r[0] = np.nan
        rows["nan_first"] = r
        r = g.standard_normal(n).astype(np.float32)
        r[5] = np.inf
        rows["pinf"] = r
        r = g.standard_normal(n).astype(np.float32)
        r[::3] = -np.inf
        rows["some_ninf"] = r
        rows["all_ninf"] = np.full(n, -np.inf, np.float32)
    return rows


def _same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or np.array_equal(a, b, equal_nan=True)


needs_ref = pytest.mark.skipif(not Reference.available(), reason="oracle/_ref not built")


@needs_ref
@pytest.mark.parametrize("n", [1, 2, 9, 1000, 40000])
def test_oracle_sample_matches_reference(oracle, n):
    ref = Reference()
    for name, row in _rows(n, 7 + n).items():
        for t in (1.0, 0.7, 0.3, 2.5, 1e-3, 0.0, -1.0):
            for seed in (1, 2, 3):
                a = row.copy()
                LIBC.srand(seed)
                if t > 0:
                    ref.lib.vec_scale(a.ctypes.data, np.float32(1.0) / np.float32(t), n)
                tr = ref.lib.sample_temperature(a.ctypes.data, n, t)
                LIBC.srand(seed)
                r = np.float32(np.float32(LIBC.rand()) / np.float32(RAND_MAX))
                to, b = oracle.sample(row, t, r)
                assert to == tr, (name, t, seed)
                assert _same(a, b), (name, t, seed)


def test_sample_hand_cases(oracle):
    x = np.array([0.0, 1.0, 2.0, 3.0], np.float32)
    assert oracle.sample(x, 1.0, 0.0)[0] == 0                  # r = 0: the first index
    assert oracle.sample(x, 1.0, 1.0)[0] in (2, 3)             # r = 1: where the running sum reaches 1
    assert oracle.sample(np.array([5.0], np.float32), 0.7, 0.9)[0] == 0
    assert oracle.sample(np.array([1.0, np.nan, 2.0], np.float32), 1.0, 0.1)[0] == 2    # NaN: n - 1
    assert oracle.sample(np.array([np.nan, 1.0, 2.0], np.float32), 0.0, 0.1)[0] == 0    # greedy: NaN first
    assert oracle.sample(np.array([1.0, 3.0, 3.0], np.float32), 0.0, 0.1)[0] == 1       # greedy: first max
    # a draw equal to a running-sum value selects that index; the next float up, the next index
    g = np.random.default_rng(5)
    x = g.standard_normal(3000).astype(np.float32)
    t = np.float32(0.7)
    _, w = oracle.sample(x, t, 0.5)
    s = np.add.accumulate(w, dtype=np.float32)[-1]
    cum = np.add.accumulate(w / s, dtype=np.float32)
    for i in (0, 1, 17, 1500, 2998):
        if cum[i] > (cum[i - 1] if i else 0):
            assert oracle.sample(x, t, cum[i])[0] == i
            up = np.nextafter(cum[i], np.float32(2))
            assert oracle.sample(x, t, up)[0] == int(np.argmax(cum >= up))
