"""Extract the grids of the IQ1_S / IQ1_M, IQ2_XS, IQ2_S, IQ3_XXS and IQ3_S
formats from the reference into a JSON fixture, and write the C tables the
oracle and the HIP library compile from it.

Runs only where the reference checkout exists (read as text, never imported
or executed).  Each grid is read from two independent copies:

* the Swift tables: ``LLM/Quantize/IQ1Grid.swift:8`` (``gpu``, 2048 x u32),
  ``LLM/Quantize/IQ3Grid.swift:5`` (``xs2``, 512 x u64), ``:136`` (``s2``,
  1024 x u64), ``:395`` (``xxs3``, 256 x u32), ``:441`` (``s3``, 512 x u32);
* the Metal header emitted from them, ``LLM/metal/IQTables.h:5``
  (``iq1s_grid_gpu``), ``:439`` (``iq2xs_grid_u32``, low word first),
  ``:613`` (``iq2s_grid_u32``), ``:958`` (``iq3xxs_grid``), ``:1004``
  (``iq3s_grid``).

It refuses to write anything unless both copies agree.  ``--inc`` (re)writes
``oracle/iq_grids.inc`` and ``chatokf_amd/csrc/iq_grids.inc`` from the JSON.
"""
import json
import os
import re
import sys

REF = os.environ.get("OKF_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
JSON = os.path.join(HERE, "iq_grids.json")

# name: (swift file, swift pattern, metal pattern, entries, bits)
GRIDS = {
    "iq1s": ("LLM/Quantize/IQ1Grid.swift", r"static let gpu: \[UInt32\] = \[",
             r"constant uint iq1s_grid_gpu\[2048\] = \{", 2048, 32),
    "iq2xs": ("LLM/Quantize/IQ3Grid.swift", r"static let xs2: \[UInt64\] = \[",
              r"constant uint iq2xs_grid_u32\[1024\] = \{", 512, 64),
    "iq2s": ("LLM/Quantize/IQ3Grid.swift", r"static let s2: \[UInt64\] = \[",
             r"constant uint iq2s_grid_u32\[2048\] = \{", 1024, 64),
    "iq3xxs": ("LLM/Quantize/IQ3Grid.swift", r"static let xxs3: \[UInt32\] = \[",
               r"constant uint iq3xxs_grid\[256\] = \{", 256, 32),
    "iq3s": ("LLM/Quantize/IQ3Grid.swift", r"static let s3: \[UInt32\] = \[",
             r"constant uint iq3s_grid\[512\] = \{", 512, 32),
}


def _array(text, start_pat):
    m = re.search(start_pat, text)
    if not m:
        raise SystemExit(f"pattern not found: {start_pat}")
    body = text[m.end():]
    end = body.index("}" if "{" in start_pat else "]")
    return [int(t, 0) for t in re.findall(r"0x[0-9a-fA-F]+|\d+", body[:end])]


def extract():
    metal = open(os.path.join(REF, "LLM/metal/IQTables.h")).read()
    out = {"source": "Swift grids (LLM/Quantize/IQ1Grid.swift:8, IQ3Grid.swift:5,136,395,441) == "
                     "LLM/metal/IQTables.h:5,439,613,958,1004"}
    for name, (sf, sp, mp, n, bits) in GRIDS.items():
        sw = _array(open(os.path.join(REF, sf)).read(), sp)
        me = _array(metal, mp)
        if len(sw) != n:
            raise SystemExit(f"{name}: {len(sw)} entries, expected {n}")
        if bits == 64:
            split = []
            for v in sw:
                split += [v & 0xFFFFFFFF, v >> 32]
            ok = split == me
        else:
            ok = sw == me
        if not ok:
            raise SystemExit(f"{name}: Swift and IQTables.h disagree")
        out[name] = [f"0x{v:0{bits // 4}x}" for v in sw]
    with open(JSON, "w") as f:
        json.dump(out, f, indent=0)
    print("wrote", JSON)


def write_inc():
    g = json.load(open(JSON))
    for path, prefix, note in [
            (os.path.join(ROOT, "oracle/iq_grids.inc"), "okf_ref_",
             "the oracle's copy"),
            (os.path.join(ROOT, "chatokf_amd/csrc/iq_grids.inc"), "okf_host_",
             "uploaded to device memory by the context")]:
        lines = ["/* Grids of IQ1_S / IQ1_M, IQ2_XS, IQ2_S, IQ3_XXS and IQ3_S (ggml format",
                 " * data, as carried by LLM/Quantize/IQ1Grid.swift and IQ3Grid.swift),",
                 f" * {note}.  Written by tests/golden/make_iq_grids.py from",
                 " * tests/golden/iq_grids.json; tests compare the two. */"]
        for name, (_, _, _, n, bits) in GRIDS.items():
            ctype, suf = ("uint64_t", "ull") if bits == 64 else ("uint32_t", "u")
            vals = [v + suf for v in g[name]]
            lines.append(f"static const {ctype} {prefix}{name}_grid[{n}] = {{")
            per = 4 if bits == 64 else 6
            for i in range(0, n, per):
                lines.append("    " + ", ".join(vals[i:i + per]) + ",")
            lines.append("};")
        with open(path, "w") as f:
            f.write("\n".join(lines) + "\n")
        print("wrote", path)


if __name__ == "__main__":
    if "--inc" not in sys.argv[1:] or "--extract" in sys.argv[1:]:
        extract()
    write_inc()
