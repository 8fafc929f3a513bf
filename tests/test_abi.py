"""CPU checks of the C-ABI boundary (no device work): the shared library
loads, exports every entry point include/glm53_moe.h declares, the Python
binding types every one of them, struct layouts agree between the header
and ctypes, and the product refuses to run without a GPU instead of falling
back to a CPU path."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from conftest import ROOT, submodule

HEADER = ROOT / "include" / "glm53_moe.h"
PACKAGE_DIR = ROOT / "glm53-flash-mlx_amd"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(glm53_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def header_define(name: str) -> int:
    m = re.search(rf"#define\s+{name}\s+(\d+)", HEADER.read_text())
    assert m, name
    return int(m.group(1))


@pytest.fixture(scope="module")
def N():
    return submodule("_native")


@pytest.fixture(scope="module")
def libso(N):
    if not N.LIB_PATH.exists():
        pytest.fail(f"{N.LIB_PATH} not built: run __graft_entry__.build() first")
    return N.load_library()


def test_header_declares_the_path_entry_points():
    names = declared_functions()
    for required in ("glm53_fp8_linear", "glm53_router_topk", "glm53_decode_moe", "glm53_decode_moe_ex",
                     "glm53_route_plan", "glm53_grouped_linear", "glm53_activate_gate_up",
                     "glm53_restore_and_reduce", "glm53_direct_order_reduce", "glm53_prefill_moe"):
        assert required in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol(libso):
    for name in declared_functions():
        assert hasattr(libso, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(submodule("_native").LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(glm53_\w+)$", out, flags=re.M))
    assert set(declared_functions()) <= exported
    # nothing glm53_* leaks out of the library that the header does not declare
    assert exported - set(declared_functions()) == set()


def test_binding_types_every_declared_symbol(N):
    assert set(N.EXPORTED_SYMBOLS) == set(declared_functions())


def test_abi_version_and_constants(N, libso):
    assert libso.glm53_abi_version() == header_define("GLM53_ABI_VERSION")
    assert libso.glm53_last_error() == b""
    assert (N.OK, N.INVALID_ARGUMENT, N.BAD_STATE, N.DEVICE_ERROR) == tuple(
        header_define(n) for n in ("GLM53_OK", "GLM53_INVALID_ARGUMENT", "GLM53_BAD_STATE", "GLM53_DEVICE_ERROR"))
    assert (N.REDUCE_GROUPED, N.REDUCE_DIRECT) == (header_define("GLM53_REDUCE_GROUPED"),
                                                   header_define("GLM53_REDUCE_DIRECT"))
    assert (N.STAGE_ROUTER, N.STAGE_GATE_UP, N.STAGE_DOWN, N.STAGE_ALL) == tuple(
        header_define(n) for n in ("GLM53_STAGE_ROUTER", "GLM53_STAGE_GATE_UP", "GLM53_STAGE_DOWN",
                                   "GLM53_STAGE_ALL"))


def test_struct_layouts_match_header(N, tmp_path):
    """sizeof / offsetof of every public struct, compiled from the header with
    the host C compiler, equal the ctypes mirrors."""
    structs = {"glm53_bank": N.Bank, "glm53_linear": N.Linear, "glm53_shared_expert": N.SharedExpert,
               "glm53_router": N.Router, "glm53_plan_counters": N.PlanCounters}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        cname, field, value = line.split()
        got[(cname, field)] = int(value)
    for cname, py in structs.items():
        assert got[(cname, "sizeof")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)


def test_invalid_arguments_fail_before_any_device_work(N, libso):
    """Status 1 (invalid argument, -> ValueError) with a message from
    glm53_last_error, for argument checks that run before any device call
    (the reference raises ValueError / std::invalid_argument for shape and
    layout errors)."""
    P = ctypes.c_void_p
    h = ctypes.c_void_p()
    cases = [
        (lambda: libso.glm53_prefill_plan_create(100, 256, 0, 32, 8, 64, 10.0, ctypes.byref(h)), "block-aligned"),
        (lambda: libso.glm53_prefill_plan_create(4096, 1536, 100, 32, 8, 64, 10.0, ctypes.byref(h)), "multiple of 128"),
        (lambda: libso.glm53_prefill_plan_create(512, 256, 0, 32, 40, 64, 10.0, ctypes.byref(h)), "top_k"),
        (lambda: libso.glm53_decode_plan_create(4096, 1536, 1536, 288, 0, 10.0, ctypes.byref(h)), "top_k"),
        (lambda: libso.glm53_decode_plan_create(4096, 1536, 1536, 288, 8, 10.0, None), "out is null"),
        (lambda: libso.glm53_split_activations(P(16), 4, 100, 100, P(16), P(16), P(16), None), "multiple of 128"),
        (lambda: libso.glm53_restore_and_reduce(P(16), P(16), P(16), 4, 0, 256, None, P(16), None), "dimensions"),
        (lambda: libso.glm53_router_topk(None, P(16), 4, P(16), P(16), P(16), 1 << 20, None), "router is null"),
        (lambda: libso.glm53_grouped_linear(P(16), 8, None, 8, 100, P(16), P(16), P(16), 1, P(16), P(16), None, 1,
                                            128, P(16), P(16), 1 << 20, None), "block-aligned"),
        (lambda: libso.glm53_decode_moe_bound_routed(None, P(16), P(16), P(16), P(16), None), "plan is null"),
        (lambda: libso.glm53_decode_moe_bound(None, P(16), P(16), None), "plan is null"),
        (lambda: libso.glm53_decode_moe_ex(None, P(16), None, None, P(16), None, P(16), 4, None), "plan is null"),
        (lambda: libso.glm53_decode_plan_counters(None, P(16)), "null pointer"),
        (lambda: libso.glm53_prefill_plan_counters(None, P(16)), "null pointer"),
        (lambda: libso.glm53_decode_plan_identities(None, 0, None, 0, P(16)), "null pointer"),
        (lambda: libso.glm53_prefill_plan_identities(None, None, 0, P(16)), "null pointer"),
    ]
    def grouped(experts, top_k, n_group, topk_group):  # a router struct with fake (never read) pointers
        return ctypes.byref(N.Router(16, 16, experts, 64, top_k, 1.0, 1, n_group, topk_group))

    cases += [
        (lambda: libso.glm53_router_topk(grouped(288, 8, 7, 2), P(16), 0, P(16), P(16), P(16), 1 << 20, None),
         "groups of two or more"),
        (lambda: libso.glm53_router_topk(grouped(288, 8, 8, 9), P(16), 0, P(16), P(16), P(16), 1 << 20, None),
         "exceeds n_group"),
        (lambda: libso.glm53_router_topk(grouped(32, 8, 8, 1), P(16), 0, P(16), P(16), P(16), 1 << 20, None),
         "kept groups"),
        (lambda: libso.glm53_router_topk(grouped(256, 8, 128, 8), P(16), 0, P(16), P(16), P(16), 1 << 20, None),
         "at most 64"),
    ]
    for call, fragment in cases:
        assert call() == N.INVALID_ARGUMENT, fragment
        assert fragment in libso.glm53_last_error().decode(), (fragment, libso.glm53_last_error())
        with pytest.raises(ValueError):
            N.check(N.INVALID_ARGUMENT)
    assert libso.glm53_split_activations(P(16), 0, 128, 128, P(16), P(16), P(16), None) == N.OK  # empty: no work
    # zero-filled group fields (a caller built against the struct without them) select ungrouped
    assert libso.glm53_router_topk(grouped(288, 8, 0, 0), P(16), 0, P(16), P(16), P(16), 1 << 20, None) == N.OK


def test_float32_gate_refuses_unsupported_groups():
    """Float32Gate(n_group, topk_group) takes what the kernels take and
    raises ValueError otherwise (the reference forwards both to
    group_expert_select, patch.py:134-142)."""
    import torch

    from conftest import pkg

    M = pkg()
    w, b = torch.zeros(288, 64), torch.zeros(288)
    M.Float32Gate(w, b, top_k=8, n_group=8, topk_group=4)
    for n_group, topk_group, top_k in ((7, 2, 8), (8, 9, 8), (8, 0, 8), (96, 8, 8), (8, 1, 37)):
        with pytest.raises(ValueError):
            M.Float32Gate(w, b, top_k=top_k, n_group=n_group, topk_group=topk_group)
    with pytest.raises(ValueError):
        M.Float32Gate(torch.zeros(7, 64), torch.zeros(7), top_k=2, n_group=7, topk_group=1)  # groups of one


def test_product_refuses_cpu_tensors():
    """No CPU fallback: a product op on host tensors raises."""
    torch = pytest.importorskip("torch")
    fp8 = submodule("fp8")
    x = torch.zeros((1, 256), dtype=torch.bfloat16)
    w = torch.zeros((128, 256), dtype=torch.uint8)
    s = torch.ones((1, 2), dtype=torch.float32)
    with pytest.raises((RuntimeError, ValueError)):
        fp8.block_fp8_linear(x, w, s)


def test_missing_library_fails_loudly(N, tmp_path):
    with pytest.raises(RuntimeError, match="missing"):
        N.load_library(tmp_path / "absent.so")


def test_product_does_not_import_the_oracle():
    for path in PACKAGE_DIR.rglob("*"):
        if path.suffix in (".py", ".cpp", ".hip", ".h"):
            text = path.read_text()
            assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.M), path
            assert "glm53o_" not in text, path


def test_bound_decode_refuses_x_of_another_dtype_or_device(N):
    """DecodePlan.execute_bound / execute_bound_router check x against the
    bound weights before any native call: BF16 only (a float32 or float16 x
    of H elements would otherwise be read as BF16 bytes), on the weights'
    device.  Exercised on a plan object without a native handle."""
    import torch

    packed = submodule("packed")
    plan = object.__new__(packed.DecodePlan)
    plan._bound = (None, [torch.empty(8, dtype=torch.uint8, device="meta")], [], 0)
    with pytest.raises(ValueError, match="bfloat16"):
        plan._check_x(torch.zeros(4096, dtype=torch.float32, device="meta"), "execute_bound")
    with pytest.raises(ValueError, match="bound weights are on meta"):
        plan._check_x(torch.zeros(4096, dtype=torch.bfloat16), "execute_bound")
    plan._check_x(torch.zeros(4096, dtype=torch.bfloat16, device="meta"), "execute_bound")


def test_abi_version_two_and_layout_constants(N, libso):
    """ABI 2: glm53_bank gained row_group_log2 and the layout entry points."""
    assert libso.glm53_abi_version() == 2 == N.ABI_VERSION
    assert (N.ROWS_LAYOUT, N.TILED_LAYOUT, N.MAX_ROW_GROUP_LOG2) == (
        0, header_define("GLM53_TILED_ROW_GROUP_LOG2"), header_define("GLM53_MAX_ROW_GROUP_LOG2"))


def test_layout_entry_points_refuse_bad_arguments_without_device_work(N, libso):
    """glm53_relayout_weights / glm53_bank_create / glm53_bank_import check
    layouts and shapes before touching a device (status 1 on this GPU-less
    host): overlap, an exponent out of range, a row-group layout of a width
    that is not a multiple of 128 or of a partial group."""
    import ctypes

    P = ctypes.c_void_p
    a, b = P(1 << 20), P((1 << 20) + 64)  # never dereferenced: refused before any device call
    assert libso.glm53_relayout_weights(a, b, 1, 16, 128, 0, 4, None) == N.INVALID_ARGUMENT
    assert "overlap" in libso.glm53_last_error().decode()
    far = P(1 << 30)
    assert libso.glm53_relayout_weights(a, far, 1, 16, 128, 0, 9, None) == N.INVALID_ARGUMENT
    assert libso.glm53_relayout_weights(a, far, 1, 16, 200, 0, 4, None) == N.INVALID_ARGUMENT
    assert "cols % 128" in libso.glm53_last_error().decode()
    assert libso.glm53_relayout_weights(a, far, 1, 24, 128, 0, 4, None) == N.INVALID_ARGUMENT
    assert "row group" in libso.glm53_last_error().decode()
    bank = N.Bank(1 << 20, 1 << 21, 1 << 22, 1 << 23, 4, 256, 129, 0, 4)  # I = 129 cannot be tiled
    out = ctypes.POINTER(N.Bank)()
    assert libso.glm53_bank_create(ctypes.byref(bank), None, ctypes.byref(out)) == N.INVALID_ARGUMENT
    assert "multiples of 128" in libso.glm53_last_error().decode()
    bank.intermediate, bank.row_group_log2 = 128, 8
    assert libso.glm53_bank_create(ctypes.byref(bank), None, ctypes.byref(out)) == N.INVALID_ARGUMENT
    bank.row_group_log2 = 0
    assert libso.glm53_bank_import(ctypes.byref(bank), 9, None, ctypes.byref(out)) == N.INVALID_ARGUMENT
    assert not out
