"""The device sigmoid's edge table (mlx-serve_amd/csrc/sigmoid_edges.h) is what its
generator writes today, ascending, and every entry equals the oracle's bf16 sigmoid table
(the correctly rounded sigmoid over all bf16 inputs). Which inputs the device routes to it
is checked on the GPU by the exhaustive SwiGLU test."""
import os
import re
import subprocess
import sys

import numpy as np

import oracle as O

CSRC = os.path.join(os.path.dirname(__file__), "..", "mlx-serve_amd", "csrc")


def _entries(text):
    """Both tables' entries, near then tail, each ascending."""
    out = []
    for name in ("Near", "Tail"):
        i = text.index(f"kSigmoidEdges{name}[")
        body = text[text.index("{", i):text.index("};", i)]
        ent = np.array([int(x, 16) for x in re.findall(r"0x([0-9A-F]{8})u", body)],
                       dtype=np.uint64)
        assert ent.size > 0 and np.all(np.diff(ent) > 0)
        out.append(ent)
    return np.concatenate(out)


def test_header_is_generator_output():
    out = subprocess.run([sys.executable, os.path.join(CSRC, "gen_sigmoid_edges.py")],
                         capture_output=True, text=True, check=True).stdout
    with open(os.path.join(CSRC, "sigmoid_edges.h")) as f:
        assert f.read() == out


def test_entries_match_oracle_table():
    with open(os.path.join(CSRC, "sigmoid_edges.h")) as f:
        ent = _entries(f.read())
    table = O.sigmoid_table_bf16()
    keys, vals = (ent >> 16).astype(np.int64), (ent & 0xFFFF).astype(np.uint16)
    assert np.array_equal(table[keys], vals)
    # every listed input is near a midpoint or in the v < -80 tail
    v = O.bf16_to_f32(keys.astype(np.uint16))
    assert np.all((v < -80) | (np.abs(v) < 80))
