import os, sys, pathlib
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
  config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libferrite_hip.so")


@pytest.fixture(scope="session")
def cuda():
  import torch
  if not torch.cuda.is_available(): pytest.skip("no GPU")
  from ferrite_amd import lib
  lib.load()  # the native library must be there: no fallback
  return torch.device("cuda:0")
