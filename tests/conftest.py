import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mlx-bun_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libmlxq.so")


@pytest.fixture(scope="session")
def O():
    """The CPU oracle (built on first use)."""
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def mlxq_dev():
    """libmlxq initialised on device 0 (fails loudly without a GPU or library)."""
    import mlxq

    mlxq.ensure_init(0)
    return mlxq


def half_ulp(ref, dtype):
    """Half a unit in the last place of T at |ref| (the rounding of an fp32
    result to the output dtype T)."""
    if dtype is None or dtype == 10:
        return np.zeros_like(np.asarray(ref, dtype=np.float64))
    mant = 7 if dtype == 12 else 10  # stored mantissa bits of bf16 / f16
    a = np.maximum(np.abs(np.asarray(ref, dtype=np.float64)), 2.0 ** -14)
    return 0.5 * 2.0 ** (np.floor(np.log2(a)) - mant)


# worst |err| / tol of every assert_close call, reported at the end of the run
HEADROOM = []


def assert_close(got, ref, atol=1e-2, rtol=1e-3, what="", dtype=None):
    """|got - ref| <= atol + rtol |ref| (+ half an ulp of T when the output is
    rounded to T = `dtype`): the attention / matmul bar against the fp32
    reference -- fp32 accumulation within max-abs 1e-2 and relative 1e-3,
    then the one rounding every T-typed output carries.  Returns the worst
    |err| / tol (1.0 = at the bar) and records it for the run summary."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    tol = atol + rtol * np.abs(ref) + half_ulp(ref, dtype)
    ratio = float((err / tol).max()) if err.size else 0.0
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0].split("::")[-1]
    HEADROOM.append((test, what, ratio, float(err.max()) if err.size else 0.0))
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} elements out of tolerance; worst at {i}: "
                             f"got {got[i]} ref {ref[i]} (max abs err {err.max():.3g}, worst err/tol {ratio:.3f})")
    return ratio


def pytest_terminal_summary(terminalreporter):
    """Per test, the worst err/tol ratio of its assert_close checks."""
    if not HEADROOM:
        return
    worst = {}
    for test, what, ratio, err in HEADROOM:
        if test not in worst or ratio > worst[test][1]:
            worst[test] = (what, ratio, err)
    terminalreporter.section("parity headroom: worst |err| / tol per test (1.0 = at the bar)")
    for test, (what, ratio, err) in sorted(worst.items(), key=lambda kv: -kv[1][1]):
        terminalreporter.write_line(f"{ratio:6.3f}  max|err| {err:.3g}  {test}  [{what}]")


def write_safetensors(path, tensors, metadata=None):
    """Write a safetensors file: tensors maps name -> (dtype string, shape,
    raw bytes) (the format of src/safetensors.ts: u64 LE header length, JSON
    header, data)."""
    import json
    import struct

    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hb = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + b"".join(blobs))
