"""Copy the reference's Q8_0 / Q4_K golden files into tests/golden/dataref/.

The files are test data of the reference (SharpMind.Tests/DataRef/, written
by tools/ReferenceDataGenerator from .NET Random(42) inputs): dtype 8 = Q8_0,
dtype 12 = Q4_K; ref_* hold the VecDot result for 4 blocks x column c,
refread_* the dequantised values.  They are copied verbatim so the GPU box
(which has no reference checkout) can run the same pins.
"""
import os
import shutil
import sys

SRC = os.path.join(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", "SharpMind.Tests", "DataRef")
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dataref")
FILES = ["seed.txt"] + [f"{k}_{d}_c{c}.bin" for k in ("ref", "refread") for d in (8, 12) for c in (0, 1)]

if __name__ == "__main__":
    os.makedirs(DST, exist_ok=True)
    for f in FILES:
        shutil.copyfile(os.path.join(SRC, f), os.path.join(DST, f))
        print("copied", f)
