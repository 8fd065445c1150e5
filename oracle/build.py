"""Builds the oracle's C restatement (oracle/bfp_c.c) into oracle/_build/liboracle_bfp.so with gcc: test
infrastructure (the checker of the full-width parity tests), compiled by __graft_entry__.build() beside the HIP
library, never linked into the product.

python -m oracle.build"""
import os, pathlib, shutil, subprocess

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle_bfp.so"


def build():
  cc = shutil.which("gcc") or shutil.which("cc")
  if cc is None: raise RuntimeError("gcc not found: the oracle's C restatement needs a C compiler")
  LIB.parent.mkdir(exist_ok=True)
  tmp = LIB.with_suffix(".so.tmp")
  # (OpenMP shares a matrix's runs among the host's cores; each run's arithmetic is independent of the others')
  r = subprocess.run([cc, "-O3", "-fopenmp", "-shared", "-fPIC", "-std=c11", "-Wall", str(HERE / "bfp_c.c"), "-o", str(tmp), "-lm"],
                     capture_output=True, text=True)
  if r.returncode: raise RuntimeError(f"gcc failed on oracle/bfp_c.c:\n{r.stderr}")
  os.replace(tmp, LIB)
  return LIB


if __name__ == "__main__":
  print(build())
