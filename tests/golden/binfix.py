"""Reader for the reference's fixture files (format of tools/gen_gdn_fixture.py:18-22): int32 n_arrays,
then per array an int32 length followed by that many little-endian float32 values."""

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent


def load(name: str) -> list[np.ndarray]:
    raw = (GOLDEN / name).read_bytes()
    n = int(np.frombuffer(raw, "<i4", 1, 0)[0])
    off = 4
    arrays = []
    for _ in range(n):
        length = int(np.frombuffer(raw, "<i4", 1, off)[0])
        off += 4
        arrays.append(np.frombuffer(raw, "<f4", length, off).copy())
        off += 4 * length
    assert off == len(raw), f"{name}: trailing bytes"
    return arrays
