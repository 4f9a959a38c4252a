"""The C ABI library: it loads, exports every function include/persistent_lstm_hip.h declares, and its
host-side logic (geometry rules, sizes, argument validation) behaves - no device work on the CPU."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from persistent_lstm_hip_amd.extension import (PLH_ERR_INVALID, PLH_ERR_UNSUPPORTED, PLH_OK, LIB_PATH,
                                               load_extension, load_error)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "persistent_lstm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(plh_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def ext():
    e = load_extension()
    assert e is not None, load_error()
    return e


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("plh_forward", "plh_pack_regressor", "plh_workspace_bytes", "plh_packed_bytes", "plh_supports",
                 "plh_status", "plh_repeat_first_row", "plh_last_error", "plh_abi_version"):
        assert must in names


def test_every_declared_symbol_is_exported(ext):
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (plh_[a-z0-9_]+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    for n in declared_functions():
        assert hasattr(ext.lib, n)


def test_abi_version_and_error_text(ext):
    assert ext.lib.plh_abi_version() == 1
    assert ext.lib.plh_supports(5, 4096, 4, 24) == 0
    assert "hidden_size" in ext.last_error()
    assert ext.lib.plh_supports(5, 1024, 4, 24) == 1 and ext.lib.plh_supports(300, 256, 2, 6) == 1


@pytest.mark.parametrize("I,H,L,O,ok", [
    (5, 128, 4, 24, True), (5, 1, 1, 1, True), (32, 32, 2, 0, True), (64, 64, 8, 3, True), (128, 128, 1, 24, True),
    (5, 129, 4, 24, True), (5, 256, 4, 24, True), (5, 512, 4, 24, True), (300, 300, 2, 1, True),
    # the reference's generic entry point serves 1 <= H <= 1024 and any input size
    # (model.py:154-165, persistent_lstm_hip.cu:2981-2991): H 513..1024 and I > padded H run layer by layer
    (5, 513, 4, 24, True), (5, 1024, 4, 24, True), (300, 256, 2, 6, True), (33, 32, 2, 4, True),
    (257, 256, 2, 4, True), (1000, 600, 1, 3, True), (4096, 1024, 2, 1, True),
    (5, 1025, 4, 24, False), (70000, 128, 1, 1, False), (0, 128, 4, 24, False), (5, 128, 0, 24, False),
    (5, 128, 4, -1, False),
])
def test_supported_geometries(ext, I, H, L, O, ok):
    assert ext.supports(I, H, L, O) is ok


def test_packed_bytes_closed_form(ext):
    # wpack (the all-layers kernels, HP <= 512 and I <= HP): L * (HP/16 waves) * (2*HP/32 chunks) * 4 gates
    # * 64 lanes * 16 B; then f32 bias, head; all 256-aligned.  The layer-sequential path (HP >= 512, or
    # I > HP with HP raised to 128 at least) adds its W_hh fragments (4HP x HP fp16 per layer), W_ih of every
    # layer its projection GEMM computes ([4HP][K padded to 128]: layer 0 only when I > 32 or HP < 512)
    # and, when layer 0's projection runs in its recurrent kernel (HP >= 512, I <= 32), layer 0's W_ih as
    # MFMA fragments (HP x 128 fp16).
    a = lambda v: (v + 255) // 256 * 256  # noqa: E731
    r128 = lambda v: (v + 127) // 128 * 128  # noqa: E731
    for I, H, L, O, HP in [(5, 128, 4, 24, 128), (5, 100, 2, 3, 128), (5, 40, 3, 7, 64), (5, 10, 1, 0, 32),
                           (5, 256, 4, 24, 256), (5, 200, 2, 3, 256), (5, 512, 4, 24, 512), (7, 400, 1, 1, 512),
                           (40, 300, 3, 2, 512), (5, 1024, 4, 24, 1024), (5, 600, 2, 3, 1024), (300, 1000, 2, 1, 1024),
                           (300, 256, 2, 6, 256), (33, 32, 2, 4, 128), (1000, 600, 1, 3, 1024), (200, 130, 3, 2, 256)]:
        wave_ok = HP <= 512 and I <= HP
        rec_ok = HP >= 512 or I > HP
        x0 = rec_ok and HP >= 512 and I <= 32
        wp = L * (HP // 16) * (HP // 16) * 4 * 64 * 16
        want = (a(wp) if wave_ok else 0) + a(L * 4 * HP * 4) + a(O * HP * 4) + a(O * 4)
        if rec_ok:
            kp0 = 0 if x0 else r128(I)
            want += a(L * 4 * HP * HP * 2) + a(4 * HP * (kp0 + (L - 1) * r128(H)) * 2)
            if x0:
                want += a(HP * 128 * 2)
        assert ext.packed_bytes(I, H, L, O) == want, (I, H, L, O)
    with pytest.raises(ValueError):
        ext.packed_bytes(5, 1025, 4, 24)


def test_workspace_bytes_grow_with_sequence(ext):
    a = ext.workspace_bytes(5, 128, 4, 24, 512, 100)
    b = ext.workspace_bytes(5, 128, 4, 24, 512, 1000)
    assert 0 < a < b
    # hand-off buffer dominates: (L-1) * rows * T * H * 2 bytes
    assert b >= 3 * 512 * 1000 * 128 * 2
    with pytest.raises(ValueError):
        ext.workspace_bytes(5, 128, 4, 24, -1, 10)


def test_sliced_workspace_layout(ext):
    # H > 128: the hidden units of a layer are split over several workgroups ("slices").  The workspace
    # holds the (L-1)-layer hand-off plus a two-step ring of tagged words per (layer, tile) through which
    # the slices exchange h every step: L * tiles * 2 * (HP * 8) words of 8 bytes, and 8 more words per
    # (layer, tile) for the slices' XCD ids; each (layer, tile) progress counter has a 128-byte line
    # of its own.  Without a device the
    # plan assumes 256 co-resident workgroups: 256 / (L * 4 slices) = 16 workgroups per layer at
    # HP = 256, each carrying two 16-row tiles (the whole 512-row batch), and 256 / (L * 16) = 4
    # one-tile workgroups at HP = 512 (a 64-row batch: one launch, where the wavefront path is the
    # faster one).
    L, T = 4, 1000
    for H, tiles, batch in ((256, 32, 512), (512, 4, 64)):
        rows = tiles * 16
        b = ext.workspace_bytes(5, H, L, 24, batch, T)
        handoff = (L - 1) * rows * T * H * 2
        ring = L * tiles * (2 * H * 8 + 8) * 8  # + a table of up to 16 slices' XCD ids per (layer, tile)
        xp = rows * T * 8 * 2  # x of the launch: one 8-wide K group (I = 5) per row and step
        counters = L * tiles * 128  # one 128-byte line per (layer, tile)
        assert handoff + ring + xp + counters <= b < handoff + ring + xp + counters + (1 << 12)


def test_layer_sequential_workspace_layout(ext):
    # HP = 512 with a batch that needs several wavefront launches (8 of 64 rows here) runs layer by
    # layer: 8 workgroups per 16-row tile hold one layer's W_hh, so 256 / 8 = 32 tiles (512 rows) fit
    # one launch.  The workspace holds one layer's input projection for every
    # step (fp16 [T][rows][4HP]), two alternating fp16 layer-input buffers [T][rows][HP], one
    # layer's exchange ring (tiles * 2 * HP * 8 words of 8 bytes, then 8 u32 per tile) and, since
    # I <= 32 puts layer 0's projection inside the recurrent kernel, x as one zero-padded 32-wide
    # MFMA K chunk per row and step (64 bytes).
    L, T, H = 4, 1000, 512
    rows = 512
    b = ext.workspace_bytes(5, H, L, 24, 512, T)
    gates = T * rows * 4 * H * 2
    xs = 2 * T * rows * H * 2
    ring = (rows // 16) * (2 * H * 8 * 8 + 16 * 8)  # + the tile's table of up to 32 slices' XCD ids
    xp = rows * T * 64
    assert gates + xs + ring + xp <= b < gates + xs + ring + xp + (1 << 12)
    # I > 32: layer 0's projection is a GEMM too (x goes to the first xs buffer): no packed x
    b40 = ext.workspace_bytes(40, H, L, 24, 512, T)
    assert gates + xs + ring <= b40 < gates + xs + ring + (1 << 12)
    # a padded H (400 -> 512) is sized by HP throughout
    assert ext.workspace_bytes(5, 400, L, 24, 512, T) == b
    # sequences whose projections would exceed 24 GiB stay on the wavefront path (64 rows per launch:
    # x, the (L-1)-layer hand-off and the ring), whatever the batch
    T = 10000
    b = ext.workspace_bytes(5, H, L, 24, 512, T)
    wave = 64 * T * 8 * 2 + (L - 1) * 64 * T * H * 2 + L * 4 * (2 * H * 8 + 8) * 8 + L * 4 * 128
    assert wave <= b < wave + (1 << 12)


def test_deep_h512_stacks_go_layer_by_layer(ext):
    # One tile of the sliced path takes L x 16 workgroups at padded H 512: beyond 16 layers it would
    # not fit 256 co-resident workgroups, so the layer-sequential path (8 per tile) serves even small
    # batches.  Its workspace: one layer's projections [T][rows][4 HP], two layer-input buffers, the
    # ring of 2 tiles (32 rows) and x packed for layer 0's in-kernel projection.
    T, rows, H = 6, 32, 512
    gates = T * rows * 4 * H * 2
    xs = 2 * T * rows * H * 2
    ring = (rows // 16) * (2 * H * 8 * 8 + 16 * 8)
    xp = rows * T * 64
    for L in (17, 40, 64):
        b = ext.workspace_bytes(5, H, L, 3, 20, T)
        assert gates + xs + ring + xp <= b < gates + xs + ring + xp + (1 << 12), L
    # 16 layers still fit one sliced tile: the wavefront path keeps the small batch
    sliced = ext.workspace_bytes(5, H, 16, 3, 20, T)
    assert sliced >= 15 * 16 * T * H * 2  # the (L-1)-layer hand-off of one 16-row tile


def test_wide_hidden_and_input_workspace_layout(ext):
    # H 513..1024 (padded 1024): only the layer-sequential path; 32 slices of 32 units per 16-row tile,
    # so 256 / 32 = 8 tiles (128 rows) per launch.  I <= 32: x packed for layer 0's in-kernel projection.
    L, T, H = 2, 100, 1024
    rows = 128
    gates = T * rows * 4 * H * 2
    xs = 2 * T * rows * H * 2
    ring = (rows // 16) * (2 * H * 8 * 8 + 16 * 8)
    xp = rows * T * 64
    b = ext.workspace_bytes(5, 700, L, 3, 512, T)
    assert gates + xs + ring + xp <= b < gates + xs + ring + xp + (1 << 12)
    # an input wider than the padded H gets its own GEMM input buffer [T * rows][K padded to 128]
    b = ext.workspace_bytes(1100, 700, L, 3, 512, T)
    xin = T * rows * 1152 * 2
    assert gates + xs + ring + xin <= b < gates + xs + ring + xin + (1 << 12)
    # I = 300 > H = 256: layer by layer at padded H 256 (4 slices of 64 units per tile, so 64 tiles = 1024
    # rows per launch); x fits the first layer-input buffer (K padded to 384 > 256: its own buffer)
    rows, H = 512, 256
    b = ext.workspace_bytes(300, H, L, 6, 512, T)
    gates = T * rows * 4 * H * 2
    xs = 2 * T * rows * H * 2
    ring = (rows // 16) * (2 * H * 8 * 8 + 16 * 8)
    xin = T * rows * 384 * 2
    assert gates + xs + ring + xin <= b < gates + xs + ring + xin + (1 << 12)


def test_forward_validates_before_touching_the_device(ext):
    f = ext.lib.plh_forward
    ws = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    # unsupported geometry
    assert f(ws, 5, 1999, 4, 24, ws, 4, 4, None, None, None, None, None, None, None, None, 0, None, None, ws, 1 << 20,
             None) == PLH_ERR_UNSUPPORTED
    # missing packed weights
    assert f(None, 5, 128, 4, 24, ws, 4, 4, None, None, None, None, None, None, None, None, 0, None, None, ws, 1 << 20,
             None) == PLH_ERR_INVALID
    # probes requested without buffers
    assert f(ws, 5, 128, 4, 24, ws, 4, 4, None, None, None, None, None, None, None, None, 2, None, None, ws, 1 << 20,
             None) == PLH_ERR_INVALID
    # misaligned workspace
    assert f(ws, 5, 128, 4, 24, ws, 4, 4, None, None, None, None, None, None, None, None, 0, None, None,
             ctypes.c_void_p(258), 1 << 20, None) == PLH_ERR_INVALID
    assert ext.lib.plh_repeat_first_row(None, None, -1, 3, None) == PLH_ERR_INVALID
    assert ext.lib.plh_repeat_first_row(None, None, 0, 0, None) == PLH_OK


def test_pack_validates_before_touching_the_device(ext):
    p = ext.lib.plh_pack_regressor
    arr = (ctypes.c_void_p * 4)()
    assert p(5, 128, 4, 24, arr, arr, arr, None, None, None, None, 0, None) == PLH_ERR_INVALID
    assert p(5, 128, 4, 24, arr, arr, arr, None, None, None, ctypes.c_void_p(256), 1 << 30, None) == PLH_ERR_INVALID
    assert p(5, 256 * 8, 4, 24, arr, arr, arr, None, None, None, None, 0, None) == PLH_ERR_UNSUPPORTED


def test_mfma_probe_validates_before_touching_the_device(ext):
    assert ext.lib.plh_probe_mfma_f16(None, None) == PLH_ERR_INVALID
    assert b"required" in ext.lib.plh_last_error()


def test_kernel_timing_arming_without_forwards(ext):
    assert ext.lib.plh_kernel_timing(0) == PLH_OK
    ms, n = ext.kernel_timing_read()
    assert n == 0 and ms == 0.0
    assert ext.lib.plh_kernel_timing(-1) == PLH_ERR_INVALID
