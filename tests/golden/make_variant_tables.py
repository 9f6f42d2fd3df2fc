"""Writes the codebooks of the IQ2_XS, IQ2_S and IQ3_S formats.

Reads the reference's table file as text
(/root/reference/src/metal_src/iq2_tables.metal:86-541: iq2xs_grid[512],
iq2s_grid[1024] as u64 of eight magnitudes, iq3s_grid[512] as u32 of four)
and writes:

  tests/golden/reference_variant_tables.json
      the values and SHA-256 digests of their little-endian images (data only);
  oracle/iq_variants_oracle_tables.h
      the oracle's copy in a compact form;
  candelora-metal-kernels_amd/csrc/iq_variants_format.h (the CODES macros)
      the kernels' copy in the same compact form.

Compact form: the IQ2 grids hold magnitudes {8, 25, 43}, stored as a u16 whose
bit pair [2j+1:2j] is the level code of byte j; the IQ3_S grid holds odd
magnitudes 1..15, stored as a u16 whose bits [3j+2:3j] give (value - 1) / 2 of
byte j.  tests/test_oracle_variants.py decodes both copies and compares them
with the digests.  No reference code is run.

Run from the repository root: `python tests/golden/make_variant_tables.py`.
"""

import hashlib
import json
import os
import re
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF_TABLES = "/root/reference/src/metal_src/iq2_tables.metal"
LEVELS2 = [8, 25, 43]


def parse_table(src: str, name: str):
    i = src.index(", %s," % name)
    j = src.index("\n", i)
    k = src.index("GGML_TABLE_END()", j)
    return [int(t, 0) for t in re.split(r"[,\s]+", src[j:k]) if t.strip()]


def code2(g: int) -> int:
    c = 0
    for j in range(8):
        c |= LEVELS2.index((g >> (8 * j)) & 0xFF) << (2 * j)
    return c


def code3(g: int) -> int:
    c = 0
    for j in range(4):
        v = (g >> (8 * j)) & 0xFF
        assert v % 2 == 1 and 1 <= v <= 15, v
        c |= ((v - 1) // 2) << (3 * j)
    return c


def fmt_codes(codes, per_line=8, indent="    "):
    lines = []
    for i in range(0, len(codes), per_line):
        lines.append(indent + ", ".join("0x%04x" % c for c in codes[i:i + per_line]) + ",")
    return lines


def main():
    src = open(REF_TABLES).read()
    xs = parse_table(src, "iq2xs_grid")
    s2 = parse_table(src, "iq2s_grid")
    s3 = parse_table(src, "iq3s_grid")
    assert (len(xs), len(s2), len(s3)) == (512, 1024, 512)
    doc = {
        "source": "src/metal_src/iq2_tables.metal:86-541 (values read as text)",
        "iq2xs_grid": ["0x%016x" % g for g in xs],
        "iq2s_grid": ["0x%016x" % g for g in s2],
        "iq3s_grid": ["0x%08x" % g for g in s3],
        "sha256": {
            "iq2xs_grid": hashlib.sha256(b"".join(struct.pack("<Q", g) for g in xs)).hexdigest(),
            "iq2s_grid": hashlib.sha256(b"".join(struct.pack("<Q", g) for g in s2)).hexdigest(),
            "iq3s_grid": hashlib.sha256(b"".join(struct.pack("<I", g) for g in s3)).hexdigest(),
        },
    }
    with open(os.path.join(HERE, "reference_variant_tables.json"), "w") as f:
        json.dump(doc, f, indent=1)
        f.write("\n")

    cx = [code2(g) for g in xs]
    cs = [code2(g) for g in s2]
    c3 = [code3(g) for g in s3]

    oracle_h = [
        "/*",
        " * TEST INFRASTRUCTURE ONLY — the oracle's own copy of the IQ2_XS, IQ2_S and",
        " * IQ3_S codebooks (ggml's iq2xs_grid, iq2s_grid, iq3s_grid as carried by the",
        " * reference at src/metal_src/iq2_tables.metal:86-541).  Compact form of this",
        " * build: IQ2 entries are u16 with bit pair [2j+1:2j] = level code of byte j",
        " * (levels {8, 25, 43}); IQ3_S entries are u16 with bits [3j+2:3j] = (v-1)/2 of",
        " * byte j.  Written by tests/golden/make_variant_tables.py; the decoded images",
        " * are pinned by SHA-256 in tests/test_oracle_variants.py.",
        " */",
        "#ifndef IQ_VARIANTS_ORACLE_TABLES_H",
        "#define IQ_VARIANTS_ORACLE_TABLES_H",
        "#include <stdint.h>",
        "",
        "static const uint16_t ORACLE_IQ2XS_CODES[512] = {",
        *fmt_codes(cx),
        "};",
        "",
        "static const uint16_t ORACLE_IQ2S_CODES[1024] = {",
        *fmt_codes(cs),
        "};",
        "",
        "static const uint16_t ORACLE_IQ3S_CODES[512] = {",
        *fmt_codes(c3),
        "};",
        "",
        "#endif",
        "",
    ]
    with open(os.path.join(REPO, "oracle", "iq_variants_oracle_tables.h"), "w") as f:
        f.write("\n".join(oracle_h))

    def macro(name, codes):
        out = ["#define %s \\" % name]
        body = fmt_codes(codes)
        for i, line in enumerate(body):
            out.append(line + (" \\" if i + 1 < len(body) else ""))
        return out

    pkg_h = [
        "// iq_variants_format.h — codebooks of the IQ2_XS, IQ2_S and IQ3_S formats.",
        "//",
        "// The grids are format data (the reference carries them as iq2xs_grid,",
        "// iq2s_grid and iq3s_grid, src/metal_src/iq2_tables.metal:86-541).  Held here",
        "// in this build's compact form: an IQ2 entry is a u16 whose bit pair",
        "// [2j+1:2j] is the level code of byte j (levels {8, 25, 43}); an IQ3_S entry",
        "// is a u16 whose bits [3j+2:3j] give (v - 1) / 2 of byte j (v odd, 1..15).",
        "// Written by tests/golden/make_variant_tables.py.",
        "#pragma once",
        "",
        *macro("CMK_IQ2XS_GRID_CODES", cx),
        "",
        *macro("CMK_IQ2S_GRID_CODES", cs),
        "",
        *macro("CMK_IQ3S_GRID_CODES", c3),
        "",
    ]
    with open(os.path.join(REPO, "candelora-metal-kernels_amd", "csrc", "iq_variants_format.h"), "w") as f:
        f.write("\n".join(pkg_h))
    print("wrote reference_variant_tables.json, iq_variants_oracle_tables.h, iq_variants_format.h")


if __name__ == "__main__":
    main()
