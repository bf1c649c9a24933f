"""The product path has no CPU fallback: every torch-facing op rejects host tensors before it reaches a library, and
the loader refuses a library that has not been built (runs without a GPU)."""
import inspect
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "reax-engine-kernels_amd"))
from reax_fmha import abi, ops  # noqa: E402

# every public op that launches work (splitkv_workspace_bytes only sizes a buffer)
OPS = [name for name, fn in inspect.getmembers(ops, inspect.isfunction)
       if not name.startswith("_") and fn.__module__ == ops.__name__ and name != "splitkv_workspace_bytes"]


def test_every_launching_op_is_listed():
    assert {"fmha_q", "fmha_b", "fmha_qp", "attention", "attention_varlen", "attention_splitkv",
            "attention_splitkv_noalloc", "rarn", "conv_l2", "conv_v", "kkt", "howu", "howu_norm", "gemm", "slices",
            "gv"} <= set(OPS)


@pytest.mark.parametrize("name", OPS)
def test_host_tensors_are_refused_before_any_library_call(name, monkeypatch):
    def no_library():
        raise AssertionError(f"{name} reached a library with host tensors")

    for loader in ("howu", "post", "plain", "slices", "gv"):
        if hasattr(abi, loader):
            monkeypatch.setattr(abi, loader, no_library)
    fn = getattr(ops, name)
    host = torch.zeros((2, 2, 2, 2), dtype=torch.bfloat16)
    args, kwargs = [], {}
    for p in inspect.signature(fn).parameters.values():
        if p.default is not inspect.Parameter.empty:
            continue
        if p.kind == inspect.Parameter.KEYWORD_ONLY:
            kwargs[p.name] = host
        else:
            args.append(host)
    with pytest.raises(ValueError, match="device tensors only"):
        fn(*args, **kwargs)


def test_loader_refuses_a_missing_library(tmp_path):
    missing = str(tmp_path / "libreax_howu.so")
    with pytest.raises(RuntimeError, match="not built"):
        abi._load(missing, abi.HOWU_SYMBOLS)
