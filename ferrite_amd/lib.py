"""ctypes binding of libferrite_hip.so (include/ferrite_hip.h), in the way ferrite binds libttsim (ferrite/pci.py:18-31):
explicit argtypes and restype for every entry point, a status code turned into an exception with the library's own
message. Pointers are plain integers (a torch tensor's data_ptr()), streams the raw hipStream_t (a torch stream's
cuda_stream). Loading fails loudly when the library is missing: there is no CPU fallback."""
import ctypes, os, pathlib

HERE = pathlib.Path(__file__).resolve().parent
PATH = pathlib.Path(os.environ.get("FERRITE_HIP_LIB", HERE / "libferrite_hip.so"))

F32, BF16, BFP8, BFP4, I32, BF16_T16 = 0, 1, 2, 3, 4, 5
AXIS_N, AXIS_K = 0, 1
EP_STORE, EP_RESIDUAL, EP_SILU_GATE, EP_ROPE_KV, EP_PROGRAM = 0, 1, 2, 3, 4
MAX_OPS, MAX_INPUTS = 15, 8
OPND_ACC, OPND_IMM = 24, 25
OPS = ["add", "sub", "mul", "max", "cmplt", "cmpne", "keep", "drop", "relu", "exp", "exp2", "log", "log2", "sin", "cos",
       "recip", "sqrt", "ftob", "itof", "ftoi", "copy"]
OP = {name: i for i, name in enumerate(OPS)}
REDUCE_SUM, REDUCE_MAX = 0, 1
DTYPES = {"fp32": F32, "bf16": BF16, "bfp8": BFP8, "bfp4": BFP4, "int32": I32}
ERRORS = {-1: ValueError, -2: NotImplementedError, -3: RuntimeError}

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_int64
S = ctypes.c_size_t


class Program(ctypes.Structure):
  """fh_program (include/ferrite_hip.h): at most 15 elementwise ops over at most 8 strided inputs."""
  _fields_ = [("n_ops", ctypes.c_int32), ("n_inputs", ctypes.c_int32), ("op", ctypes.c_int8 * 16), ("a", ctypes.c_int8 * 16),
              ("b", ctypes.c_int8 * 16), ("imm", ctypes.c_float * 16), ("input", P * MAX_INPUTS),
              ("in_dtype", ctypes.c_int32 * MAX_INPUTS), ("in_stride", (L * 3) * MAX_INPUTS)]


class Epilogue(ctypes.Structure):
  """fh_epilogue (include/ferrite_hip.h)."""
  _fields_ = [("kind", I), ("norm_w", P), ("ssq_in", P), ("eps", ctypes.c_float), ("centered", I),
              ("residual", P), ("ssq_out", P), ("split", I), ("heads", I), ("kv_heads", I), ("head_dim", I),
              ("cos_tab", P), ("sin_tab", P), ("places", P), ("cache_rows", P), ("cache", P), ("cache_dtype", I),
              ("cache_len", L), ("argmax_parts", P), ("program", ctypes.POINTER(Program)), ("copy_bf16", P), ("copy_w", P),
              ("rope_rows", L), ("copy_tiles", I)]


SIGNATURES = {
  "fh_last_error": ([], ctypes.c_char_p),
  "fh_version": ([], ctypes.c_char_p),
  "fh_bfp_bytes": ([L, L, I, I, ctypes.POINTER(S), ctypes.POINTER(S)], I),
  "fh_bfp_pack": ([P, I, L, L, L, I, I, P, P, P], I),
  "fh_bfp_dequant": ([P, P, L, L, I, I, P, L, P], I),
  "fh_gemv_bfp": ([P, I, L, I, L, L, P, P, I, ctypes.POINTER(Epilogue), P, I, L, P], I),
  "fh_gemv_bfp_k": ([P, I, L, I, L, L, P, P, I, ctypes.POINTER(Epilogue), P, I, L, P], I),
  "fh_gemm_bfp": ([P, I, L, L, L, L, P, P, I, ctypes.POINTER(Epilogue), P, I, L, P], I),
  "fh_matmul": ([P, I, L, L, P, I, L, L, L, L, L, L, ctypes.POINTER(Program), P, I, L, L, P], I),
  "fh_embed_rows": ([P, I, L, L, P, I, P, P, P], I),
  "fh_attention_workspace_bytes": ([I, I, I, L], S),
  "fh_kv_cache_bytes": ([I, I, L, I], S),
  "fh_attention_decode": ([P, P, I, L, I, I, I, I, P, P, L, P, I, P, S, P], I),
  "fh_attention_decode_noalloc": ([P, P, I, L, I, I, I, I, P, P, L, P, I, P], I),
  "fh_attention_prefill": ([P, L, P, I, L, I, I, I, I, L, L, P, I, L, P], I),
  "fh_rms_rows": ([P, L, L, L, P, ctypes.c_float, I, P, I, L, P], I),
  "fh_moe_route": ([P, L, I, L, P, ctypes.c_float, I, P, I, I, I, I, P, P, P, P], I),
  "fh_moe_workspace_bytes": ([I, I, L, L], S),
  "fh_moe_experts": ([P, L, I, L, P, P, ctypes.c_float, I, I, L, P, P, I, P, P, I, P, P, P, P, P, S, P], I),
  "fh_map": ([ctypes.POINTER(Program), P, I, L, L, L, L, L, P], I),
  "fh_reduce": ([ctypes.POINTER(Program), I, I, L, L, L, P, I, P], I),
  "fh_softmax_rows": ([ctypes.POINTER(Program), I, L, L, L, P, I, P], I),
  "fh_argmax_rows": ([P, L, L, P, P], I),
  "fh_argmax_parts": ([P, L, L, P, P], I),
  "fh_read_probe": ([P, S, P, I, P], I),
  "fh_mfma_probe": ([I, I, P, I, P], I),
  "fh_lds_probe": ([I, P, I, P], I),
  "fh_heads_workspace_bytes": ([I, L, I], S),
  "fh_logit_heads": ([P, L, I, L, I, P, P, P, P, P, S, P], I),
  "fh_gather_cols": ([P, L, L, P, L, L, L, P, L, P], I),
  "fh_gather_rows": ([P, L, L, L, P, L, L, L, P, L, L, P], I),
  "fh_moe_touched": ([P, L, P, L, I, I, I, P, P, P], I),
  "fh_moe_group": ([P, L, I, I, I, P, P, P, P, P], I),
  "fh_attend": ([P, I, L, L, P, P, I, L, L, L, L, L, I, L, I, P, L, L, P, I, L, L, P], I),
  "fh_put_rows": ([P, L, L, L, P, L, L, L, P, L, L, P], I),
}

_lib = None


def load():
  """The library, loaded once; raises if it is not built (ferrite_amd.build) or lacks an entry point."""
  global _lib
  if _lib is None:
    if not PATH.exists(): raise RuntimeError(f"{PATH} is not built: run python -m ferrite_amd.build (needs hipcc)")
    lib = ctypes.CDLL(str(PATH))
    for name, (args, res) in SIGNATURES.items():
      fn = getattr(lib, name)
      fn.argtypes, fn.restype = args, res
    _lib = lib
  return _lib


def call(name, *args):
  """Calls an entry point that returns a status; a negative one raises with fh_last_error()'s message."""
  lib = load()
  rc = getattr(lib, name)(*args)
  if rc < 0: raise ERRORS.get(rc, RuntimeError)(lib.fh_last_error().decode())
  return rc


def bfp_bytes(K, N, fmt, axis=AXIS_N):
  m, e = S(), S()
  call("fh_bfp_bytes", K, N, fmt, axis, ctypes.byref(m), ctypes.byref(e))
  return m.value, e.value
