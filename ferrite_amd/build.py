"""Builds libferrite_hip.so in-tree: every .hip file under ferrite_amd/csrc, compiled by hipcc for gfx950.

python -m ferrite_amd.build [--jobs N]"""
import concurrent.futures, os, pathlib, shutil, subprocess, sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libferrite_hip.so"
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
         # packed fp32 ops are left to nobody: hipcc would make them from plain float code
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # a kernel's leading scalar arguments arrive in SGPRs with its waves (gfx950 kernel-argument preloading), so
         # the first loads of the hot kernels do not wait on the argument buffer
         "-mllvm", "-amdgpu-kernarg-preload-count=16",
         "-I", str(HERE.parent / "include")]


def hipcc():
  path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
  if not os.path.exists(path): raise RuntimeError("hipcc not found: ROCm is needed to build libferrite_hip.so")
  return path


def build(jobs=None, verbose=False):
  """Compiles each source to an object in ferrite_amd/_build, links them into ferrite_amd/libferrite_hip.so."""
  out = HERE / "_build"
  out.mkdir(exist_ok=True)
  sources = sorted(CSRC.glob("*.hip"))
  cc = hipcc()
  def compile_one(src):
    obj = out / (src.stem + ".o")
    cmd = [cc, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode: raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    if verbose and r.stderr.strip(): print(r.stderr, file=sys.stderr)
    return obj
  with concurrent.futures.ThreadPoolExecutor(jobs or min(8, len(sources))) as ex:
    objs = list(ex.map(compile_one, sources))
  tmp = LIB.with_suffix(".so.tmp")
  r = subprocess.run([cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)], capture_output=True, text=True)
  if r.returncode: raise RuntimeError(f"link failed:\n{r.stderr}")
  os.replace(tmp, LIB)
  return LIB


if __name__ == "__main__":
  jobs = int(sys.argv[sys.argv.index("--jobs") + 1]) if "--jobs" in sys.argv else None
  print(build(jobs, verbose=True))
