"""Write reference_tables.json: the numeric tables of the reference that the
step engine must reproduce, read as data from the reference sources.

  kickoff_permutations  src/RLConstants.cu:4-29         [120][4] spawn order
  kickoff_locations     include/RLConstants.cuh:51-57   x, y, yaw / (pi/4)
  respawn_locations     include/RLConstants.cuh:59-64   x, y, yaw / (pi/2)
  boost_pads            include/Physics/BoostPads.cuh:21-56   x, y, z, big

Run from the repository root with the reference checked out at
/root/reference:  python tests/golden/make_reference_tables.py
"""
import json
import re
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).with_name("reference_tables.json")


def block(text: str, start: str) -> str:
    i = text.index(start)
    j = text.index("};", i)
    return text[i:j]


def main() -> None:
    consts = (REF / "src/RLConstants.cu").read_text()
    perms = [[int(v) for v in m.groups()] for m in
             re.finditer(r"\{\s*(\d)\s*,\s*(\d)\s*,\s*(\d)\s*,\s*(\d)\s*\}", block(consts, "KICKOFF_PERMUTATIONS"))]
    header = (REF / "include/RLConstants.cuh").read_text()
    spawn = r"\{\s*(-?[\d.]+)f\s*,\s*(-?[\d.]+)f\s*,\s*CAR_REST_Z\s*,\s*PI_(\d)\s*\*\s*(\d)\s*\}"
    kick = [[float(x), float(y), int(k)] for x, y, _, k in re.findall(spawn, block(header, "KICKOFF_LOCATIONS"))]
    resp = [[float(x), float(y), int(k)] for x, y, _, k in re.findall(spawn, block(header, "RESPAWN_LOCATIONS"))]
    pads_src = (REF / "include/Physics/BoostPads.cuh").read_text()
    pad = r"\{\{\s*(-?[\d.]+)f\s*,\s*(-?[\d.]+)f\s*,\s*(-?[\d.]+)f\s*\}\s*,\s*(BIG|SMALL)_PAD_RADIUS"
    pads = [[float(x), float(y), float(z), int(kind == "BIG")] for x, y, z, kind in
            re.findall(pad, block(pads_src, "BOOST_PADS[NUM_BOOST_PADS]"))]
    assert len(perms) == 120 and len(kick) == 5 and len(resp) == 4 and len(pads) == 34
    OUT.write_text(json.dumps({
        "source": "jwmccarthy/CARL src/RLConstants.cu, include/RLConstants.cuh, include/Physics/BoostPads.cuh",
        "kickoff_permutations": perms,
        "kickoff_locations": kick,
        "respawn_locations": resp,
        "boost_pads": pads,
    }) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
