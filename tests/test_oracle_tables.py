"""Pins the oracle's (and the kernels') codebook tables.

Checks, independent of each other:
  * SHA-256 of the little-endian images equal the digests recorded from the
    reference text (kmask 5ac9831b..., ksigns a76742a6..., grid 05826b5d...);
  * the tables equal the values in tests/golden/reference_tables.json (read from
    the reference's table file) and, where /root/reference exists, the live text;
  * closed forms: kmask[j] = 1 << j, ksigns[i] = i | parity(i) << 7;
  * grid invariants: 256 unique entries, ascending, every byte in {8, 25, 43};
  * the product's compact codebook (csrc/iq2xxs_format.h) decodes to the same grid.
"""

import hashlib
import json
import os
import re
import struct

import numpy as np
import pytest

from conftest import PKG_DIR, REPO

GOLDEN = os.path.join(REPO, "tests", "golden", "reference_tables.json")
SHA_PREFIX = {
    "kmask_iq2xs": "5ac9831b2e30eb28",
    "ksigns_iq2xs": "a76742a603f8beca",
    "iq2xxs_grid": "05826b5d3e472a3a",
}


def _images(oracle):
    km, ks, gr = oracle.tables()
    return km, ks, gr, {
        "kmask_iq2xs": hashlib.sha256(km.tobytes()).hexdigest(),
        "ksigns_iq2xs": hashlib.sha256(ks.tobytes()).hexdigest(),
        "iq2xxs_grid": hashlib.sha256(b"".join(struct.pack("<Q", int(g)) for g in gr)).hexdigest(),
    }


def test_sha256_of_tables(oracle):
    _, _, _, h = _images(oracle)
    for k, prefix in SHA_PREFIX.items():
        assert h[k].startswith(prefix), k


def test_tables_equal_reference_values(oracle):
    km, ks, gr, h = _images(oracle)
    doc = json.load(open(GOLDEN))
    assert list(km) == doc["kmask_iq2xs"]
    assert list(ks) == doc["ksigns_iq2xs"]
    assert [int(g) for g in gr] == [int(v, 16) for v in doc["iq2xxs_grid"]]
    for k in SHA_PREFIX:
        assert h[k] == doc["sha256"][k]


@pytest.mark.skipif(not os.path.exists("/root/reference/src/metal_src/iq2_tables.metal"),
                    reason="reference checkout not present")
def test_tables_equal_live_reference_text(oracle):
    src = open("/root/reference/src/metal_src/iq2_tables.metal").read()

    def parse(name):
        i = src.index(", %s," % name)
        j = src.index("\n", i)
        k = src.index("GGML_TABLE_END()", j)
        return [int(t, 0) for t in re.split(r"[,\s]+", src[j:k]) if t.strip()]

    km, ks, gr = oracle.tables()
    assert list(km) == parse("kmask_iq2xs")
    assert list(ks) == parse("ksigns_iq2xs")
    assert [int(g) for g in gr] == parse("iq2xxs_grid")


def test_closed_forms(oracle):
    km, ks, gr = oracle.tables()
    assert [int(v) for v in km] == [1 << j for j in range(8)]
    for i in range(128):
        assert ks[i] == (i | ((bin(i).count("1") & 1) << 7))
        assert bin(int(ks[i])).count("1") % 2 == 0  # even parity of every sign byte


def test_grid_invariants(oracle):
    _, _, gr = oracle.tables()
    vals = [int(g) for g in gr]
    assert len(set(vals)) == 256
    assert vals == sorted(vals)
    for g in vals:
        assert {(g >> (8 * j)) & 0xFF for j in range(8)} <= {8, 25, 43}
    assert vals[0] == 0x0808080808080808  # index 0 is all 8s


def test_product_codebook_matches_oracle(oracle):
    """The kernels' compact codebook (macro CMK_IQ2XXS_GRID_CODES) decodes to the
    same 256 entries."""
    src = open(os.path.join(PKG_DIR, "csrc", "iq2xxs_format.h")).read()
    i = src.index("#define CMK_IQ2XXS_GRID_CODES")
    j = src.index("\n\n", i)
    codes = [int(t, 16) for t in re.findall(r"0x[0-9a-fA-F]+", src[i:j])]
    assert len(codes) == 256
    levels = [8, 25, 43]
    decoded = []
    for c in codes:
        v = 0
        for jj in range(8):
            v |= levels[(c >> (2 * jj)) & 3] << (8 * jj)
        decoded.append(v)
    _, _, gr = oracle.tables()
    assert decoded == [int(g) for g in gr]
    assert np.all(np.array(codes) >> 16 == 0)
