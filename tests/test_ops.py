"""The registered torch ops and the C-ABI struct, without a GPU: op names and schemas (declared mutations), fake
(meta) propagation as torch.compile sees it, and wkv7_args' field order and offsets in the header, the library and
the ctypes binding."""
import os
import re

import pytest

from conftest import REPO

torch = pytest.importorskip("torch")

from rwkv_next_amd import _lib  # noqa: E402
from rwkv_next_amd import kernels  # noqa: E402
from torch._subclasses.fake_tensor import FakeTensorMode  # noqa: E402


def schema(op):
    return op.default._schema


def test_reference_op_name_is_registered_with_the_reference_schema():
    """rwkv_next::wkv7_fwd(Tensor r, w, k, v, a, b, Tensor h0, int H, int K, bool final) -> (Tensor, Tensor),
    functional (rwkv_next/kernels/wkv7.py:113-123)."""
    for op in (torch.ops.rwkv_next.wkv7_fwd, torch.ops.rwkv_next_amd.wkv7_fwd):
        s = schema(op)
        assert [a.name for a in s.arguments] == ["r", "w", "k", "v", "a", "b", "h0", "H", "K", "final"]
        assert not any(a.alias_info and a.alias_info.is_write for a in s.arguments)
        assert len(s.returns) == 2


def test_in_place_ops_declare_their_mutations():
    s = schema(torch.ops.rwkv_next_amd.wkv7_pool_)
    written = {a.name for a in s.arguments if a.alias_info and a.alias_info.is_write}
    assert written == {"pool", "snapshots", "status"}
    s = schema(torch.ops.rwkv_next_amd.wkv7_replay_)
    written = {a.name for a in s.arguments if a.alias_info and a.alias_info.is_write}
    assert written == {"state"}
    assert len(s.returns) == 0


def test_fake_propagation():
    with FakeTensorMode():
        x = torch.empty(3, 5, 8 * 64, dtype=torch.bfloat16, device="cuda")
        xt = torch.empty(3, 8 * 64, 5, dtype=torch.bfloat16, device="cuda").transpose(1, 2)  # strided v
        pool = torch.empty(7, 8, 64, 64, device="cuda")
        slots = torch.empty(3, dtype=torch.int64, device="cuda")
        o, ht = torch.ops.rwkv_next.wkv7_fwd(x, x, x, xt, x, x, pool[:0], 8, 64, True)
        assert o.shape == (3, 5, 512) and o.is_contiguous() and o.dtype == torch.bfloat16
        assert ht.shape == (3, 8, 64, 64) and ht.dtype == torch.float32
        o, ht = torch.ops.rwkv_next_amd.wkv7_fwd(x, x, x, x, x, x, pool[:3], 8, 64, False)
        assert ht.numel() == 0
        o = torch.ops.rwkv_next_amd.wkv7_pool_(x, x, x, x, x, x, pool, slots, 8, 64, None, None, None, True, True,
                                              None, None, 0, 0, -1)
        assert o.shape == x.shape and o.device.type == "cuda"
        o = torch.ops.rwkv_next_amd.wkv7_pool_(x, x, x, x, x, x, pool, slots, 8, 64, None, None, None, True, False,
                                              None, None, 0, 0, -1)
        assert o.numel() == 0
        assert torch.ops.rwkv_next_amd.wkv7_replay_(x, x, x, x, x, x, pool[:3], slots, 8, 64) is None


def header_fields():
    text = open(os.path.join(REPO, "include", "wkv7.h")).read()
    body = re.search(r"typedef struct wkv7_args \{(.*?)\} wkv7_args;", text, flags=re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        for part in decl.split(","):
            names.append(re.findall(r"(\w+)\s*$", part.strip())[0])
    return names


def test_wkv7_args_field_order_and_offsets():
    binding = [name for name, _ in _lib.Wkv7Args._fields_]
    assert header_fields() == binding
    assert _lib.args_layout() == _lib.binding_layout()
    assert binding[-1] == "status"


def test_status_bits_match_header():
    text = open(os.path.join(REPO, "include", "wkv7.h")).read()
    for name in ("H0_SLOT", "HT_SLOT", "SEQLENS", "NKEEP", "DECAY", "SLOT_CLASH", "CLASH_MAX_SEQS", "SEGMENT_WAIT"):
        value = int(re.search(rf"#define WKV7_STATUS_{name} (\d+)", text).group(1))
        assert value == getattr(_lib, f"WKV7_STATUS_{name}")
    from rwkv_next_amd.kernels.wkv7 import STATUS_REASONS
    assert set(STATUS_REASONS) == {1, 2, 4, 8, 16, 32, 64}
    for name in ("AUTO", "RECURRENT", "CHUNKED", "CHAIN", "SEGMENTED"):
        value = int(re.search(rf"#define WKV7_ALGO_{name} (\d+)", text).group(1))
        assert value == getattr(_lib, f"ALGO_{name}")
    w_max = float(re.search(r"#define WKV7_CHUNK_W_MAX ([0-9.]+)f", text).group(1))
    assert w_max == _lib.WKV7_CHUNK_W_MAX
    flag = re.search(r"#define WKV7_SEG_FLAG_BYTES \((\d+)u << (\d+)\)", text)
    assert int(flag.group(1)) << int(flag.group(2)) == _lib.WKV7_FLAG_REGION_BYTES
