"""Copies the reference's own golden data files into tests/golden/.

The four .npz archives are the JAX-generated fixtures that GraphGP.jl's test suite reads
(test/reference/*.npz, written by test/dump_reference.py and test/python_parity_*.py in the
reference; MIT licence, (c) Benjamin Dodge & Philipp Frank). They are data (inputs and expected
outputs), copied byte for byte; run this once where the reference checkout is available.
"""
import os
import shutil
import sys

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/test/reference"
DST = os.path.dirname(os.path.abspath(__file__))

for name in ("small.npz", "medium.npz", "generate_parity.npz", "aniso_parity.npz"):
    shutil.copyfile(os.path.join(SRC, name), os.path.join(DST, name))
    print("copied", name)
