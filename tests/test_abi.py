"""The C ABI: libmlora.so loads, exports every entry point include/mlora.h declares, and the
ctypes signatures agree with the header; host-side argument checks (CPU only, no kernel runs)."""

import ctypes
import re

import pytest
import torch

from conftest import ROOT

HEADER = ROOT / "include" / "mlora.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(mlora_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        params = [p for p in m.group(2).replace("\n", " ").split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_the_header_declares_the_entry_points():
    names = declared()
    assert {"mlora_grouped_gemm", "mlora_grouped_reduce", "mlora_route_topk", "mlora_route_sort", "mlora_tile_map",
            "mlora_last_error"} <= set(names)


def test_the_library_exports_every_declared_symbol():
    from meepsquared_amd import _lib

    lib = ctypes.CDLL(str(_lib.LIBRARY))
    for name in declared():
        assert hasattr(lib, name), name


def test_the_ctypes_signatures_match_the_header():
    from meepsquared_amd._lib import SIGNATURES

    names = declared()
    assert set(SIGNATURES) == set(names)
    for name, count in names.items():
        assert len(SIGNATURES[name][1]) == count, name


def test_a_refusal_reports_its_reason_without_a_gpu():
    from meepsquared_amd import _lib

    # E = 0 is refused before anything reaches the device
    args = [None, 8, 8, 8, 8,                 # x, ldx, rows, K, N
            None, 0, 64, 1, 8,                # w, dtype, strides
            None, 0, 0, 0,                    # scale
            None, None, None, None, None,     # nf4
            None, 0, 0, None, 0, 0, 0, 1.0,   # adapters, rank, scaling
            None, 0, None, 8, None, 0,        # bias, out, low
            None, 0, None]                    # offsets, E = 0, stream
    rc = _lib.lib.mlora_grouped_gemm(*args)
    assert rc != 0
    assert b"E=0" in _lib.lib.mlora_last_error()
    # one (E + 1)-bin count per chunk of 256 ids
    assert _lib.lib.mlora_route_sort_workspace_bytes(65536, 128) == 256 * 129 * 4


def test_a_mismatched_stack_is_refused():
    # tests/test_grouped.py:84-89 of the reference; the check runs on the host
    from meepsquared_amd import _grouped

    weight = torch.randn(2, 16, 32)
    with pytest.raises(ValueError, match="in=32"):
        _grouped._stack_strides(weight, 64, False)
    with pytest.raises(ValueError, match="in=16"):
        _grouped._stack_strides(weight, 64, True)


def test_the_operator_refuses_cpu_tensors():
    from meepsquared_amd import lora_linear

    x = torch.randn(8, 64, dtype=torch.bfloat16)
    w = torch.randn(2, 16, 64, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="GPU"):
        lora_linear(x, w, None, torch.tensor([4, 8], dtype=torch.int32), False)


def test_rank_padding_and_adapter_roles():
    from meepsquared_amd import _grouped

    lhs, rhs = torch.randn(3, 10, 4), torch.randn(3, 4, 12)
    a = _grouped._Adapters(lhs, rhs, False)
    assert a.at.shape == (3, 16, 12) and a.bt.shape == (3, 10, 16) and a.rank == 4
    assert torch.equal(a.at[:, :4].float(), rhs.bfloat16().float()) and not a.at[:, 4:].any()
    t = _grouped._Adapters(rhs.transpose(1, 2), lhs.transpose(1, 2), True)
    assert torch.equal(t.at, a.at) and torch.equal(t.bt, a.bt)
