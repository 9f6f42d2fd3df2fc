"""Writes the golden fixtures under tests/golden/.

  reference_tables.json  kmask_iq2xs / ksigns_iq2xs / iq2xxs_grid values read
                         from the reference's table file
                         (/root/reference/src/metal_src/iq2_tables.metal:4-84)
                         as text, plus SHA-256 digests of their little-endian
                         images.  Data only; no reference code is run.
  reference_cases.json   the reference's in-test cases (src/iq2_matmul.rs:
                         1065-1253): parity_case (m=2, N=7, K=320, tol 2e-3),
                         parity_case_w8a8 (tol 3e-3) and w8a8_smoke_case inputs
                         (seeds) with the oracle's outputs, and the f16 bits of
                         the 7x320 dequantised weights.

Run from the repository root: `python tests/golden/make_golden.py`.
The reference-table part is skipped when /root/reference is absent.
"""

import hashlib
import json
import os
import re
import struct
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import oracle  # noqa: E402

REF_TABLES = "/root/reference/src/metal_src/iq2_tables.metal"


def parse_table(src: str, name: str):
    i = src.index(", %s," % name)
    j = src.index("\n", i)
    k = src.index("GGML_TABLE_END()", j)
    return [int(t, 0) for t in re.split(r"[,\s]+", src[j:k]) if t.strip()]


def write_reference_tables():
    if not os.path.exists(REF_TABLES):
        print("reference absent; keeping existing reference_tables.json")
        return
    src = open(REF_TABLES).read()
    km = parse_table(src, "kmask_iq2xs")
    ks = parse_table(src, "ksigns_iq2xs")
    gr = parse_table(src, "iq2xxs_grid")
    doc = {
        "source": "src/metal_src/iq2_tables.metal:4-84 (values read as text)",
        "kmask_iq2xs": km,
        "ksigns_iq2xs": ks,
        "iq2xxs_grid": ["0x%016x" % g for g in gr],
        "sha256": {
            "kmask_iq2xs": hashlib.sha256(bytes(km)).hexdigest(),
            "ksigns_iq2xs": hashlib.sha256(bytes(ks)).hexdigest(),
            "iq2xxs_grid": hashlib.sha256(b"".join(struct.pack("<Q", g) for g in gr)).hexdigest(),
        },
    }
    with open(os.path.join(HERE, "reference_tables.json"), "w") as f:
        json.dump(doc, f, indent=1)


def case(m, out_dim, in_dim, bseed, sseed, tail):
    x, wb, ws = oracle.reference_case_inputs(m, out_dim, in_dim, bseed, sseed, tail)
    return x, wb, ws


def write_reference_cases():
    out = {}
    x, wb, ws = case(2, 7, 320, 0xA11CE5ED, 0xC0FFEE12, 0x5A)
    y = oracle.matmul_reference(x, 2, 7, 320, wb, ws)
    yq = oracle.matmul_reference_w8a8(x, 2, 7, 320, wb, ws)
    deq = oracle.dequantize_f16_bits(wb, ws, 7, 320)
    out["parity_case"] = {
        "m": 2, "out_dim": 7, "in_dim": 320, "bytes_seed": 0xA11CE5ED,
        "scales_seed": 0xC0FFEE12, "tail": 0x5A, "tolerance_abs": 2e-3,
        "weight_bytes_sha256": hashlib.sha256(wb.tobytes()).hexdigest(),
        "weight_scales_sha256": hashlib.sha256(ws.tobytes()).hexdigest(),
        "out_f32_bits": [int(v) for v in y.view("uint32").ravel()],
        "out_w8a8_f32_bits": [int(v) for v in yq.view("uint32").ravel()],
        "w8a8_tolerance_abs": 3e-3,
        "dequant_f16_sha256": hashlib.sha256(deq.tobytes()).hexdigest(),
        "dequant_f16_first_row": [int(v) for v in deq[0, :64]],
    }
    x, wb, ws = case(2, 6, 320, 0x0BADC0DE, 0xD15EA5ED, 0xC3)
    yq = oracle.matmul_reference_w8a8(x, 2, 6, 320, wb, ws)
    out["w8a8_smoke_case"] = {
        "m": 2, "out_dim": 6, "in_dim": 320, "bytes_seed": 0x0BADC0DE,
        "scales_seed": 0xD15EA5ED, "tail": 0xC3,
        "out_w8a8_f32_bits": [int(v) for v in yq.view("uint32").ravel()],
    }
    with open(os.path.join(HERE, "reference_cases.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    oracle.build()
    write_reference_tables()
    write_reference_cases()
    print("fixtures written to", HERE)
