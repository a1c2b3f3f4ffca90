"""Extract the IQ2_XXS tables from the reference into a JSON fixture.

Runs only where the reference checkout exists (it is read as text, never
imported or executed).  It reads two independent copies of the same tables:

* the Swift grids, ``LLM/Quantize/IQ2Grid.swift:6`` (``xxs``, 256 x u64),
  ``:73`` (``ksigns``, 128 x u8) and ``:87`` (``kmask``, 8 x u8);
* the Metal header emitted from them, ``LLM/metal/IQTables.h:350``
  (``iq2xxs_grid_u32``, the u64 grid split low word first, per
  ``LLM/Quantize/IQTablesEmit.swift:31-39``), ``:1093`` and ``:1104``.

It also reads the IQ4_NL levels from both places: ``IQ4_NL.kvalues``
(``LLM/Gemma/Gemma4Quant.swift:8-11``) and ``kvalues_iq4nl`` in the Metal
header.

It refuses to write the fixture unless both copies agree, then stores the
values (data only) in ``iq2xxs_tables.json`` next to this script.
"""
import json
import os
import re
import sys

REF = os.environ.get("OKF_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))


def _array(text, start_pat):
    m = re.search(start_pat, text)
    if not m:
        raise SystemExit(f"pattern not found: {start_pat}")
    body = text[m.end():]
    end = body.index("}" if "{" in start_pat else "]")
    return [int(t, 0) for t in re.findall(r"0x[0-9a-fA-F]+|\d+", body[:end])]


def main():
    swift = open(os.path.join(REF, "LLM/Quantize/IQ2Grid.swift")).read()
    metal = open(os.path.join(REF, "LLM/metal/IQTables.h")).read()
    grid = _array(swift, r"static let xxs: \[UInt64\] = \[")
    ksigns = _array(swift, r"static let ksigns: \[UInt8\] = \[")
    kmask = _array(swift, r"static let kmask: \[UInt8\] = \[")
    g32 = _array(metal, r"constant uint iq2xxs_grid_u32\[512\] = \{")
    ks_m = _array(metal, r"constant uchar ksigns_iq2xs\[128\] = \{")
    km_m = _array(metal, r"constant uchar kmask_iq2xs\[8\] = \{")
    assert len(grid) == 256 and len(ksigns) == 128 and len(kmask) == 8
    gemma = open(os.path.join(REF, "LLM/Gemma/Gemma4Quant.swift")).read()
    m = re.search(r"static let kvalues: \[Float\] = \[([^\]]*)\]", gemma)
    nl_swift = [int(v) for v in re.findall(r"-?\d+", m.group(1))]
    m = re.search(r"kvalues_iq4nl\[16\] = \{([^}]*)\}", metal)
    nl_metal = [int(v) for v in re.findall(r"-?\d+", m.group(1))]
    if len(nl_swift) != 16 or nl_swift != nl_metal:
        raise SystemExit("IQ4_NL levels disagree")
    split = []
    for v in grid:
        split += [v & 0xFFFFFFFF, v >> 32]
    if split != g32 or ksigns != ks_m or kmask != km_m:
        raise SystemExit("Swift grids and IQTables.h disagree")
    out = {
        "source": "LLM/Quantize/IQ2Grid.swift:6,73,87 == LLM/metal/IQTables.h:350,1093,1104",
        "iq2xxs_grid": [f"0x{v:016x}" for v in grid],
        "ksigns": ksigns,
        "kmask": kmask,
        "kvalues_iq4nl": nl_swift,
        "kvalues_iq4nl_source": "LLM/Gemma/Gemma4Quant.swift:8-11 == kvalues_iq4nl in LLM/metal/IQTables.h",
    }
    path = os.path.join(HERE, "iq2xxs_tables.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0)
    print("wrote", path)


if __name__ == "__main__":
    sys.exit(main())
