"""The lazy Tensor's fusion on the host (no GPU): which ops a realize puts in one program, and how it reads its inputs
(ferrite/tensor.py's _fit, _tree and _expr decide the same for ferrite's fused_kernel)."""
import pytest

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def T():
  from ferrite_amd import lib, tensor
  try:
    lib.load()
  except RuntimeError:
    pytest.skip("libferrite_hip.so is not built")
  return tensor


def test_chain_is_one_program(T):
  rt = T.Runtime("cpu")
  x = T.Tensor.of(rt, [[1.0, 2.0], [3.0, 4.0]], "fp32")
  y = T.Tensor.of(rt, [[0.5, 0.25]], "fp32")  # a row, broadcast down the rows
  z = ((x * 2 + y).exp() - x).relu()
  prog, inputs = T._fit_program(z, z.shape, allow_acc=True)
  assert [p[0] for p in prog] == ["mul", "add", "exp", "sub", "relu"]
  assert [t for t, _ in inputs] == [x, y]
  assert inputs[1][1] == [2, 0, 1]  # y's rows: a stride of 0
  assert prog[0] == ("mul", 16, T.lib.OPND_IMM, 2.0) and prog[1][1:3] == (0, 17) and prog[3][1:3] == (2, 16)
  assert rt.launches == 0  # planning launches nothing


def test_shared_node_is_one_register(T):
  rt = T.Runtime("cpu")
  x = T.Tensor.of(rt, [[1.0, 2.0]], "fp32")
  e = x.exp()
  prog, _ = T._fit_program(e * e + e, (1, 1, 2), allow_acc=True)
  assert [p[0] for p in prog] == ["exp", "mul", "add"]


def test_reversed_number(T):
  rt = T.Runtime("cpu")
  x = T.Tensor.of(rt, [[1.0, 2.0]], "fp32")
  prog, _ = T._fit_program(1 - x, (1, 1, 2), allow_acc=True)
  assert prog == [("sub", T.lib.OPND_IMM, 16, 1.0)]


def test_matmul_is_the_epilogue_acc(T):
  rt = T.Runtime("cpu")
  x = T.Tensor.of(rt, [[1.0] * 32], "bf16")
  w = T.Tensor(rt, 32, 48, dtype="bfp8")
  w.data = object()  # (a packed weight: planning reads only its shape)
  bias = T.Tensor.of(rt, [[0.0] * 48], "bf16")
  z = ((x @ w) + bias).relu()
  prog, inputs = T._fit_program(z, z.shape, allow_acc=True)
  assert [p[0] for p in prog] == ["add", "relu"] and prog[0][1] == T.lib.OPND_ACC
  assert [t for t, _ in inputs] == [bias]
