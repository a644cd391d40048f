"""The C ABI without a GPU: the library loads, exports every function that include/nca_hip.h
declares, its structs have the header's layout, and argument checks fail with the documented
status codes before any device work."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from ncas_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nca_hip.h")


def _declared_functions() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\**\s*(nca_[a-z_0-9]+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.library_path()):
        pytest.skip("libnca_hip.so is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_and_bindings_list_the_same_functions():
    declared = _declared_functions()
    assert len(declared) >= 10
    assert declared == set(_lib.EXPORTS)


def test_library_exports_every_declared_function(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_struct_layouts_match_the_header(tmp_path):
    """sizeof / offsetof of the header's structs, compiled with the host C compiler, against the
    ctypes mirrors."""
    structs = {"nca_cell_desc": _lib.CellDesc, "nca_cell_weights": _lib.CellWeights,
               "nca_fire_desc": _lib.FireDesc, "nca_cell_grads": _lib.CellGrads,
               "nca_bptt_loss": _lib.BpttLoss}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "nca_hip.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(out[cname]) == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert int(out[f"{cname}.{fname}"]) == getattr(cls, fname).offset, (cname, fname)


def _cell(**kw):
    d = dict(channels=64, heads=4, hidden=256, c_in=10, in_offset=0, c_out=16, out_offset=10,
             n_out=9, padding=2, head_kind=0, precision=1)
    d.update(kw)
    return _lib.CellDesc(**d)


def test_version_and_packed_sizes(lib):
    assert lib.nca_version() == 100
    for prec in (0, 1):
        n = lib.nca_packed_weights_bytes(ctypes.byref(_cell(precision=prec)))
        assert n > 0 and n % 256 == 0
    # the bf16 layout carries the extra fc2 fragment order
    assert lib.nca_packed_weights_bytes(ctypes.byref(_cell(precision=1))) > \
        lib.nca_packed_weights_bytes(ctypes.byref(_cell(precision=0))) // 2
    for bad in (dict(channels=48), dict(hidden=100), dict(heads=3), dict(n_out=40),
                dict(c_in=70), dict(padding=7), dict(precision=5)):
        assert lib.nca_packed_weights_bytes(ctypes.byref(_cell(**bad))) == 0, bad


def test_argument_errors_return_status_and_message(lib):
    cell = _cell()
    fire = _lib.FireDesc(seed=1, p_fire=0.5)
    rc = lib.nca_rollout(ctypes.byref(cell), None, 4, 9, 9, None, None, None, None,
                         ctypes.byref(fire), 8, None, None, None, None)
    assert rc == _lib.NCA_ERR_INVALID
    assert b"NULL" in lib.nca_last_error()
    rc = lib.nca_rollout(ctypes.byref(_cell(channels=48)), None, 4, 9, 9, None, None, None, None,
                         ctypes.byref(fire), 8, None, None, None, None)
    assert rc == _lib.NCA_ERR_UNSUPPORTED
    rc = lib.nca_rollout(ctypes.byref(cell), None, -1, 9, 9, None, None, None, None,
                         ctypes.byref(fire), 8, None, None, None, None)
    assert rc == _lib.NCA_ERR_INVALID
    # zero rows is a valid empty call
    assert lib.nca_rollout(ctypes.byref(cell), None, 0, 9, 9, None, None, None, None,
                           ctypes.byref(fire), 8, None, None, None, None) == _lib.NCA_OK
    assert lib.nca_step(ctypes.byref(cell), None, 2, 0, 9, None, None, None, None, None, None,
                        None) == _lib.NCA_ERR_INVALID
    assert lib.nca_fire_mask(4, 9, 9, None, 0, None, None, None, None) == _lib.NCA_ERR_INVALID
    adaptive = _lib.FireDesc(seed=1, p_fire=0.5, p_low=0.1, tau=0.9, adaptive=1)
    assert lib.nca_fire_mask(4, 9, 9, ctypes.byref(adaptive), 0, None, None,
                             ctypes.c_void_p(8), None) == _lib.NCA_ERR_INVALID
    assert b"conf_cell" in lib.nca_last_error()
    assert lib.nca_conf_select(None, None, 2, 4, 4, None, None) == _lib.NCA_ERR_INVALID
    assert lib.nca_conf_select(ctypes.c_void_p(8), None, 2, 0, 4, ctypes.c_void_p(8),
                               None) == _lib.NCA_ERR_INVALID
    assert lib.nca_set_kernel_path(7) == _lib.NCA_ERR_INVALID
    assert lib.nca_set_kernel_path(0) == _lib.NCA_OK


def test_workspace_query_and_refusal_without_workspace(lib):
    """Rows that fit the resident kernels need no workspace; a 201x201 grid needs one state
    buffer, and a multi-step call without it is refused before any device work."""
    c16 = _cell(channels=16, hidden=128, c_in=4, c_out=4, out_offset=4, n_out=4, padding=1)
    assert lib.nca_rollout_workspace_bytes(ctypes.byref(_cell()), 32768, 9, 9) == 0
    assert lib.nca_rollout_workspace_bytes(ctypes.byref(c16), 16, 201, 201) == 2 * 16 * 16 * 201 * 201 * 4
    assert lib.nca_rollout_workspace_bytes(ctypes.byref(_cell(channels=48)), 4, 9, 9) == 0
    fire = _lib.FireDesc(seed=1, p_fire=0.5)
    p = ctypes.c_void_p(1 << 20)
    rc = lib.nca_rollout_ws(ctypes.byref(c16), p, 16, 201, 201, p, p, p, ctypes.c_void_p(1 << 40),
                            ctypes.byref(fire), 3, None, None, None, None, 0, None)
    assert rc == _lib.NCA_ERR_UNSUPPORTED and b"workspace" in lib.nca_last_error()
    rc = lib.nca_rollout(ctypes.byref(c16), p, 16, 201, 201, p, p, p, ctypes.c_void_p(1 << 40),
                         ctypes.byref(fire), 3, None, None, None, None)
    assert rc == _lib.NCA_ERR_UNSUPPORTED
    assert lib.nca_set_kernel_path(2) == _lib.NCA_OK
    assert lib.nca_rollout_workspace_bytes(ctypes.byref(_cell()), 8, 9, 9) == 2 * 8 * 64 * 81 * 4
    assert lib.nca_set_kernel_path(0) == _lib.NCA_OK


def test_bptt_argument_checks(lib):
    c32 = _cell(channels=32, hidden=256, c_in=4, c_out=4, out_offset=4, n_out=2, padding=1)
    n = lib.nca_bptt_workspace_bytes(ctypes.byref(c32), 64, 30, 30, 32)
    M = 64 * 900
    # bf16, 32 channels, 256 hidden units: the fused MLP backward (z, g_z, g_dx, g_u, 2 x g_x)
    assert 4 * M * (2 * 128 + 4 * 32) <= n < 4 * M * (2 * 128 + 2 * 256 + 4 * 32)
    c32f = _cell(channels=32, hidden=256, c_in=4, c_out=4, out_offset=4, n_out=2, padding=1, precision=0)
    nf = lib.nca_bptt_workspace_bytes(ctypes.byref(c32f), 64, 30, 30, 32)
    assert nf >= 4 * M * (2 * 128 + 2 * 256 + 4 * 32)  # fp32 GEMM path: also h and g_a
    assert lib.nca_bptt_workspace_bytes(ctypes.byref(_cell(head_kind=1)), 4, 9, 9, 8) == 0
    assert b"mlp head" in lib.nca_last_error()
    fire = _lib.FireDesc(seed=1, p_fire=0.5)
    rc = lib.nca_bptt_backward(ctypes.byref(c32), None, None, 4, 30, 30, None, None,
                               ctypes.byref(fire), 4, None, None, None, None, None, None, 0, None)
    assert rc == _lib.NCA_ERR_INVALID and b"NULL" in lib.nca_last_error()
    adaptive = _lib.FireDesc(seed=1, p_fire=0.5, p_low=0.1, tau=0.9, adaptive=1)
    p = ctypes.c_void_p(1 << 20)
    rc = lib.nca_bptt_forward(ctypes.byref(c32), p, 4, 30, 30, p, p, p, ctypes.byref(adaptive), 4,
                              p, None)
    assert rc == _lib.NCA_ERR_UNSUPPORTED


def test_check_maps_status_to_python_exceptions(lib):
    lib.nca_set_kernel_path(9)
    with pytest.raises(ValueError):
        _lib.check(_lib.NCA_ERR_INVALID, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.NCA_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.NCA_ERR_HIP, "x")
    _lib.check(_lib.NCA_OK, "x")


def test_operators_refuse_cpu_tensors():
    """The HIP path has no CPU implementation: CPU tensors are rejected, never computed."""
    import torch

    from ncas_amd.inference import rollout_steps
    from ncas_amd.model import build_model

    m = build_model("maze_c16")
    x = torch.zeros(1, 16, 13, 13)
    g = torch.zeros(1, 1, 13, 13, dtype=torch.bool)
    c = torch.zeros(1, 4, 13, 13)
    with pytest.raises((ValueError, RuntimeError)):
        rollout_steps(m, x, g, c, 2)


def test_bptt_forward_piece_plan(lib):
    """The planning of nca_bptt_forward_ws's board pieces (host only): three pieces while every
    board's pieces fit the CUs at once, else two, else whole boards; none for grids whose pieces
    would be too short for a halo refresh, for fp32 cells (no streamed kernel) and an unsupported
    cell; the test override of the CU count (nca_set_piece_debug) replaces the device's."""
    c32 = _cell(channels=32, hidden=256, c_in=4, c_out=4, out_offset=4, n_out=2, padding=1)
    plan = lambda rows, H=30, W=30, cus=256, c=c32: lib.nca_bptt_forward_pieces(  # noqa: E731
        ctypes.byref(c), rows, H, W, cus)
    assert plan(64) == 3 and plan(85) == 3 and plan(86) == 2 and plan(128) == 2
    assert plan(129) == 1 and plan(1000) == 1
    assert plan(64, cus=128) == 2 and plan(64, cus=100) == 1
    assert plan(8, H=13, W=13) == 1  # pieces of 5 rows: too short
    assert plan(8, H=20, W=30) == 2  # 10-row pieces; thirds of 7 rows are too short
    c32f = _cell(channels=32, hidden=256, c_in=4, c_out=4, out_offset=4, n_out=2, padding=1,
                 precision=0)
    assert plan(64, c=c32f) == 1
    assert plan(64, c=_cell(channels=24)) == 0
    try:
        assert lib.nca_set_piece_debug(0, 0, 10_000) == 0
        assert plan(1000, cus=256) == 3  # the override wins
    finally:
        lib.nca_set_piece_debug(0, 0, 0)
    assert plan(1000) == 1
    assert lib.nca_set_piece_debug(-1, 0, 0) == _lib.NCA_ERR_INVALID
