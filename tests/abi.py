"""Names of the C-ABI enums, read from include/carl_amd.h (test helper)."""
from __future__ import annotations

import re
from pathlib import Path

HEADER = Path(__file__).resolve().parents[1] / "include" / "carl_amd.h"


def abi_header_text() -> str:
    return HEADER.read_text()


def enum_values(prefix: str) -> dict[str, int]:
    text = HEADER.read_text()
    return {m.group(1): int(m.group(2))
            for m in re.finditer(r"\b(" + prefix + r"[A-Z0-9_]*)\s*=\s*(-?\d+)", text)}


def field_names(prefix: str, total_key: str) -> list[str]:
    """Per-plane names: a field spanning k planes gets suffixes _0.._k-1."""
    vals = enum_values(prefix)
    total = vals.pop(total_key)
    starts = sorted((v, k) for k, v in vals.items())
    names = [""] * total
    for i, (start, name) in enumerate(starts):
        stop = starts[i + 1][0] if i + 1 < len(starts) else total
        for j in range(start, stop):
            names[j] = name if stop - start == 1 else f"{name}_{j - start}"
    return names


CAR_NAMES = field_names("CARL_CAR_", "CARL_CAR_FIELDS")
SIM_NAMES = field_names("CARL_SIM_", "CARL_SIM_FIELDS")


def declared_functions() -> list[str]:
    return re.findall(r"^\s*(?:int|void\*|void|const char\*)\s+(carl_\w+)\(", HEADER.read_text(), re.M)
