"""Copy the reference's own golden fixtures into tests/golden/ (run once, here).

The fixtures are data the reference's test-suite holds (inputs + expected
outputs as .npz, plus the manifests that record their provenance and f32
floors). They are copied byte-for-byte, never regenerated, from
`/root/reference/tests/golden/` (AdityaP9116/ARMHackathon):

  1d/            every Mamba-1 case (tests/golden/*.npz, manifest.json)
  2d/            every SS2D case (tests/golden/2d/)
  mamba3/        every SISO case captured from the official Triton kernel
                 (00-03 are L 256 at the published 24 heads x 64, dqk 128)
  mamba3_mimo/   every MIMO case captured from the official TileLang kernel
                 (00-04 and 07 at the published head shapes, 08 rank 2,
                 09 dqk 64 with 16 heads)

Nothing in the GPU tests, smoke() or bench.py reads /root/reference; they read
these copies.
"""

import shutil
import sys
from pathlib import Path

SRC = Path("/root/reference/tests/golden")
DST = Path(__file__).resolve().parent

SETS = {
    "1d": (SRC, ["*.npz", "manifest.json"]),
    "2d": (SRC / "2d", ["*.npz", "manifest.json"]),
    "mamba3": (SRC / "mamba3", ["manifest.json", "mamba3_siso_combined_*.npz"]),
    "mamba3_mimo": (SRC / "mamba3_mimo", ["manifest.json", "mamba3_mimo_combined_*.npz"]),
}


def main():
    if not SRC.is_dir():
        print(f"{SRC} not present; nothing to copy")
        return 1
    for sub, (src, pats) in SETS.items():
        out = DST / sub
        out.mkdir(parents=True, exist_ok=True)
        for pat in pats:
            for f in sorted(src.glob(pat)):
                shutil.copyfile(f, out / f.name)
                print(f"{sub}/{f.name}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
