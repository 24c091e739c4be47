"""The C ABI on the CPU: the library loads, exports exactly what
include/wal2026_amd.h declares, builds plans, and refuses malformed calls
before any launch (no GPU is touched by these tests)."""
from __future__ import annotations

import ctypes
import re
import struct
from pathlib import Path

import pytest

from wal2026_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "wal2026_amd.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^(?:int|const char\s*\*)\s*(wal_\w+)\s*\(", text, flags=re.M))


def test_header_and_binding_agree():
    assert declared_functions() == set(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    assert L.wal_abi_version() == _lib.ABI_VERSION
    assert L.wal_last_error() == b""


def _fake_layer(rows_per_group, in_features=64, S=2, K=256, id_dtype=_lib.U8, block=8, plan=None):
    groups = (_lib.WalGroup * len(rows_per_group))()
    r0 = 0
    for i, rows in enumerate(rows_per_group):
        for s in range(S):
            groups[i].stage_ids[s] = 0x100000 + 0x1000 * i + s * 16
            groups[i].codebooks[s] = 0x200000 + 0x1000 * i + s * 16
        groups[i].row_scale = 0x300000 + 0x1000 * i
        groups[i].row0 = r0
        groups[i].rows = rows
        r0 += rows
    L = _lib.WalLayer()
    L.in_features = in_features
    L.out_features = r0
    L.block_size = block
    L.blocks_per_row = -(-in_features // block)
    L.codebook_size = K
    L.num_stages = S
    L.id_dtype = id_dtype
    L.codebook_dtype = _lib.F16
    L.scale_dtype = _lib.F16
    L.scale_rows = 1
    L.n_groups = len(rows_per_group)
    L.groups = ctypes.cast(groups, ctypes.POINTER(_lib.WalGroup))
    L.plan = plan
    return L, groups


def test_plan_tables():
    L, groups = _fake_layer([256, 256, 100])
    lib = _lib.lib()
    size = ctypes.c_size_t(0)
    assert lib.wal_rvq_plan_size(ctypes.byref(L), ctypes.byref(size)) == 0
    buf = (ctypes.c_uint8 * size.value)()
    assert lib.wal_rvq_plan_build(ctypes.byref(L), buf, size.value) == 0
    raw = bytes(buf)
    magic, n_groups, goff, _ = struct.unpack_from("<4i", raw, 0)
    toff = struct.unpack_from("<3i", raw, 16)
    ntiles = struct.unpack_from("<3i", raw, 28)
    assert magic == 0x57524C31 and n_groups == 3
    # tile kinds of 16, 64 and 256 rows; tiles never straddle groups
    assert ntiles == (16 + 16 + 7, 4 + 4 + 2, 1 + 1 + 1)
    t256 = [struct.unpack_from("<4i", raw, toff[2] + 16 * i) for i in range(ntiles[2])]
    assert t256 == [(0, 0, 256, 0), (1, 0, 256, 256), (2, 0, 100, 512)]
    t16 = [struct.unpack_from("<4i", raw, toff[0] + 16 * i) for i in range(ntiles[0])]
    assert t16[-1] == (2, 96, 4, 608)
    # the group table is a verbatim copy of the host array
    g2 = raw[goff + 2 * ctypes.sizeof(_lib.WalGroup): goff + 3 * ctypes.sizeof(_lib.WalGroup)]
    assert g2 == bytes(groups[2])
    # too small a buffer is refused
    assert lib.wal_rvq_plan_build(ctypes.byref(L), buf, size.value - 1) == _lib.ESIZE


@pytest.mark.parametrize("mutate,code,needle", [
    (lambda L: setattr(L, "num_stages", 9), _lib.EINVAL, "num_stages"),
    (lambda L: setattr(L, "codebook_size", 300), _lib.EINVAL, "does not fit"),
    (lambda L: setattr(L, "out_features", 999), _lib.EINVAL, "cover"),
    (lambda L: setattr(L, "blocks_per_row", 1), _lib.EINVAL, "in_features"),
    (lambda L: setattr(L, "id_dtype", 7), _lib.EINVAL, "id dtype"),
    (lambda L: setattr(L, "scale_rows", 0), _lib.EINVAL, "scale_rows"),
])
def test_linear_refuses_bad_layers(mutate, code, needle):
    L, _g = _fake_layer([64])
    mutate(L)
    lib = _lib.lib()
    rc = lib.wal_rvq_linear(ctypes.byref(L), 0, 0, 0x1000, 1, _lib.BF16, None, _lib.F32, 0x2000, _lib.BF16, None)
    assert rc == code
    assert needle in lib.wal_last_error().decode()


def test_multi_group_needs_plan():
    L, _g = _fake_layer([64, 64])
    lib = _lib.lib()
    rc = lib.wal_rvq_reconstruct(ctypes.byref(L), 0, 0, 0x1000, _lib.BF16, None)
    assert rc == _lib.EINVAL and "plan" in lib.wal_last_error().decode()


def test_gaps_between_groups_refused():
    L, groups = _fake_layer([64, 64])
    groups[1].row0 = 65
    L.plan = 0x5000
    lib = _lib.lib()
    rc = lib.wal_rvq_reconstruct(ctypes.byref(L), 0, 0, 0x1000, _lib.BF16, None)
    assert rc == _lib.EINVAL and "starts at row" in lib.wal_last_error().decode()


def test_null_arguments_refused():
    lib = _lib.lib()
    assert lib.wal_rvq_linear(None, 0, 0, 0x1000, 1, _lib.BF16, None, _lib.F32, 0x2000, _lib.BF16, None) == _lib.EINVAL
    L, _g = _fake_layer([64])
    assert lib.wal_rvq_linear(ctypes.byref(L), 0, 0, None, 1, _lib.BF16, None, _lib.F32, 0x2000, _lib.BF16,
                              None) == _lib.EINVAL
    assert lib.wal_rvq_linear(ctypes.byref(L), 5, 0, 0x1000, 1, _lib.BF16, None, _lib.F32, 0x2000, _lib.BF16,
                              None) == _lib.EINVAL
    # m == 0 is a no-op that touches nothing
    assert lib.wal_rvq_linear(ctypes.byref(L), 0, 0, 0x1000, 0, _lib.BF16, None, _lib.F32, 0x2000, _lib.BF16,
                              None) == _lib.OK


def test_triton_matmul_feature_mismatch():
    lib = _lib.lib()
    rc = lib.wal_rvq_group_linear_matmul(0x1000, 1, 100, _lib.BF16, 0x2000, _lib.U8, 2, 64, 3, 0x3000, _lib.F16,
                                         256, 32, 0x4000, _lib.F16, 0x5000, _lib.BF16, None)
    assert rc == _lib.EINVAL and "Feature mismatch" in lib.wal_last_error().decode()


def test_id_route_argument_checks():
    lib = _lib.lib()
    rc = lib.wal_id_route_linear(0x1000, 1, 64, _lib.BF16, 0x2000, _lib.U8, 8, 0x3000, 100, _lib.F16, 0x4000,
                                 None, _lib.F32, 0, 0x5000, _lib.BF16, None)
    assert rc == _lib.EINVAL and "id dtype" in lib.wal_last_error().decode()
    rc = lib.wal_id_route_linear(0x1000, 1, 64, _lib.BF16, 0x2000, _lib.I16, 8, 0x3000, 100, _lib.F16, 0x4000,
                                 None, _lib.F32, 2, 0x5000, _lib.BF16, None)
    assert rc == _lib.EINVAL and "mode" in lib.wal_last_error().decode()


def test_image_size_and_argument_checks():
    """Codebook image bytes: per group S x K entries of 16 bytes (32 for the
    fp32 form used by multi-stage layers with stage scales or non-fp16
    codebooks); unsupported layouts and dtypes are refused on the host."""
    lib = _lib.lib()
    size = ctypes.c_size_t(0)
    L, _g = _fake_layer([64, 64], S=2, K=256, plan=0x5000)
    assert lib.wal_rvq_image_size(ctypes.byref(L), _lib.RECONSTRUCT, _lib.BF16, ctypes.byref(size)) == _lib.OK
    assert size.value == 2 * 2 * 256 * 16
    L.codebook_dtype = _lib.BF16  # multi-stage sums of bf16 codebooks are staged as fp32 values
    assert lib.wal_rvq_image_size(ctypes.byref(L), _lib.RECONSTRUCT, _lib.BF16, ctypes.byref(size)) == _lib.OK
    assert size.value == 2 * 2 * 256 * 32
    assert lib.wal_rvq_image_size(ctypes.byref(L), _lib.RECONSTRUCT_FAST, _lib.F16, ctypes.byref(size)) == _lib.OK
    assert size.value == 2 * 2 * 256 * 16
    assert lib.wal_rvq_image_size(ctypes.byref(L), _lib.RECONSTRUCT, _lib.F32, ctypes.byref(size)) == _lib.EINVAL
    L4, _g4 = _fake_layer([64], block=4)
    assert lib.wal_rvq_image_size(ctypes.byref(L4), _lib.RECONSTRUCT, _lib.BF16,
                                  ctypes.byref(size)) == _lib.EUNSUPPORTED
    # dst must be aligned and large enough (refused before any launch)
    L1, _g1 = _fake_layer([64], S=1, K=256)
    assert lib.wal_rvq_image_build(ctypes.byref(L1), 0, _lib.BF16, 0x1008, 1 << 20, None) == _lib.EINVAL
    assert lib.wal_rvq_image_build(ctypes.byref(L1), 0, _lib.BF16, 0x1000, 16, None) == _lib.ESIZE


def test_linear_refuses_mismatched_image():
    """An image built for another semantics or activation dtype is refused."""
    L, _g = _fake_layer([64], S=1, K=256)
    L.image = 0x7000
    L.image_tag = _lib.image_tag(_lib.RECONSTRUCT, _lib.F16)
    lib = _lib.lib()
    rc = lib.wal_rvq_linear(ctypes.byref(L), _lib.RECONSTRUCT, 0, 0x1000, 1, _lib.BF16, None, _lib.F32, 0x2000,
                            _lib.BF16, None)
    assert rc == _lib.EINVAL and "image" in lib.wal_last_error().decode()


def _info(L, m, x_dtype=_lib.BF16, semantics=_lib.RECONSTRUCT, x=0x8000000):
    out = _lib.WalLaunchInfo()
    rc = _lib.lib().wal_rvq_linear_info(ctypes.byref(L), semantics, x, m, x_dtype, ctypes.byref(out))
    return rc, out


def _bench_layer(rows_per_group, in_features, S, K, id_dtype, scale_rows=1):
    L, g = _fake_layer(rows_per_group, in_features=in_features, S=S, K=K, id_dtype=id_dtype,
                       plan=0x7000000 if len(rows_per_group) > 1 else None)
    L.scale_rows = scale_rows
    return L, g


# (name, groups, in, S, K, ids, scale_rows, m, x dtype) -> (x_mode, slots, grid) on a 256-CU device
PLANS = [
    ("c3_down_m1", [4096], 14336, 1, 4096, _lib.I16, 128, 1, _lib.BF16, ("lds", 2, 256)),
    ("c3_down_m2", [4096], 14336, 1, 4096, _lib.I16, 128, 2, _lib.BF16, ("lds", 1, 256)),
    ("c3_down_m3", [4096], 14336, 1, 4096, _lib.I16, 128, 3, _lib.BF16, ("lds", 1, 256)),
    ("c3_down_m4", [4096], 14336, 1, 4096, _lib.I16, 128, 4, _lib.BF16, ("global", 2, 256)),
    ("c3_down_m16", [4096], 14336, 1, 4096, _lib.I16, 128, 16, _lib.BF16, ("gtr", 1, 256)),
    ("c3_gate_up_m1", [14336, 14336], 4096, 1, 4096, _lib.I16, 128, 1, _lib.BF16, ("reg", 2, 256)),
    ("c3_gate_up_m16", [14336, 14336], 4096, 1, 4096, _lib.I16, 128, 16, _lib.BF16, ("greg", 1, 256)),
    ("c5_down_m1", [256] * 14, 18944, 3, 256, _lib.U8, 1, 1, _lib.BF16, ("lds", 2, 224)),
    ("c2_down_m1", [2048], 8192, 2, 256, _lib.U8, 1, 1, _lib.BF16, ("lds", 1, 128)),
    ("c1_m1", [2048], 2048, 2, 256, _lib.U8, 1, 1, _lib.F16, ("reg", 1, 128)),
]


@pytest.mark.parametrize("case", PLANS, ids=[p[0] for p in PLANS])
def test_decode_planner_at_benchmark_shapes(case, monkeypatch):
    """The decode launch planner's layouts at the benchmark shapes (what the
    full-size GPU tests rely on to reach each x-mode).  No GPU is needed: the
    query reads no device memory and assumes 256 CUs without a device."""
    monkeypatch.delenv("WAL2026_DECODE_XMODE", raising=False)
    _name, groups, in_f, S, K, idt, sr, m, xdt, want = case
    L, _g = _bench_layer(groups, in_f, S, K, idt, sr)
    rc, info = _info(L, m, xdt)
    assert rc == _lib.OK, _lib.lib().wal_last_error()
    assert info.kernel == _lib.KERNEL_DECODE
    assert (_lib.XMODE_NAMES[info.x_mode], info.table_slots, info.grid) == want
    assert info.lds_bytes <= 160 * 1024 and info.tile_shape == -1


def test_prefill_and_generic_routing(monkeypatch):
    monkeypatch.delenv("WAL2026_PREFILL_TILE", raising=False)
    L, _g = _bench_layer([14336], 4096, 2, 256, _lib.U8)
    rc, info = _info(L, 2048)
    assert rc == _lib.OK and info.kernel == _lib.KERNEL_PREFILL and info.tile_shape == _lib.TILE_TALL
    # 56 weight tiles x 8 x tiles, 128 k-steps each, no split
    assert info.x_mode == -1 and (info.grid, info.share, info.k_splits) == (448, 128, 1)
    monkeypatch.setenv("WAL2026_PREFILL_TILE", "wide")
    rc, info = _info(L, 2048)
    assert rc == _lib.OK and info.tile_shape == _lib.TILE_WIDE
    # block size 32, fp32 x, a misaligned x and STAGEWISE go to the generic kernel
    L32, _g32 = _fake_layer([64], in_features=256, block=32)
    assert _info(L32, 1)[1].kernel == _lib.KERNEL_GENERIC
    assert _info(L, 1, x_dtype=_lib.F32)[1].kernel == _lib.KERNEL_GENERIC
    assert _info(L, 1, x=0x8000008)[1].kernel == _lib.KERNEL_GENERIC
    assert _info(L, 1, semantics=_lib.STAGEWISE)[1].kernel == _lib.KERNEL_GENERIC
    assert _info(L, 0)[1].kernel == _lib.KERNEL_NONE


def _ws_size(L, m, x_dtype=_lib.BF16, x=0x8000000):
    n = ctypes.c_size_t(123)
    rc = _lib.lib().wal_rvq_linear_workspace_size(ctypes.byref(L), _lib.RECONSTRUCT, x, m, x_dtype, ctypes.byref(n))
    return rc, n.value


def test_prefill_split_k_plan(monkeypatch):
    """A 4096-row layer at m = 64 is 16 short tiles: with a workspace the
    planner splits each tile's 448 k-steps 16 ways (one round of 256
    workgroups, 32 k-steps each) and sizes the fp32 partials; a layer with
    enough tiles is not split; WAL2026_PREFILL_KSPLIT forces a count."""
    for v in ("WAL2026_PREFILL_TILE", "WAL2026_PREFILL_KSPLIT"):
        monkeypatch.delenv(v, raising=False)
    L, _g = _bench_layer([4096], 14336, 2, 256, _lib.U8)
    rc, info = _info(L, 64)
    assert rc == _lib.OK and info.tile_shape == _lib.TILE_SHORT
    assert (info.grid, info.share, info.k_splits) == (256, 32, 16)
    assert _ws_size(L, 64) == (_lib.OK, 16 * 64 * 4096 * 4)
    # 28672 rows: 112 tiles at m = 64, 224 with two slices; 448 tiles at m = 512 (no split)
    G, _gg = _bench_layer([28672], 4096, 2, 256, _lib.U8)
    assert (_info(G, 64)[1].k_splits, _info(G, 512)[1].k_splits) == (2, 1)
    assert _ws_size(G, 512) == (_lib.OK, 0)
    # decode rows and the generic kernel never split
    assert _ws_size(L, 16) == (_lib.OK, 0) and _info(L, 16)[1].k_splits == -1
    assert _ws_size(L, 64, x_dtype=_lib.F32) == (_lib.OK, 0)
    monkeypatch.setenv("WAL2026_PREFILL_KSPLIT", "3")
    rc, info = _info(L, 64)
    assert (info.k_splits, info.grid, info.share) == (3, 48, 8 * 19)  # 56 units of 8 steps: 19 per slice
    assert _ws_size(L, 64) == (_lib.OK, 3 * 64 * 4096 * 4)
    monkeypatch.setenv("WAL2026_PREFILL_KSPLIT", "0")
    assert _info(L, 64)[0] == _lib.EINVAL


def test_linear_ws_argument_checks():
    """wal_rvq_linear_ws refuses a misaligned or too small workspace before
    any launch (no device memory is touched)."""
    L, _g = _bench_layer([4096], 14336, 2, 256, _lib.U8)
    lib = _lib.lib()
    args = (ctypes.byref(L), _lib.RECONSTRUCT, 0, 0x8000000, 64, _lib.BF16, None, _lib.BF16, 0x9000000, _lib.BF16)
    assert lib.wal_rvq_linear_ws(*args, 0xA000004, 1 << 30, None) == _lib.EINVAL
    assert lib.wal_rvq_linear_ws(*args, 0xA000000, 1024, None) == _lib.ESIZE
    assert b"workspace" in lib.wal_last_error()


@pytest.mark.parametrize("mode", ["reg", "lds", "greg", "gtr", "global"])
def test_forced_decode_xmode(mode, monkeypatch):
    """WAL2026_DECODE_XMODE forces the x-mode wherever it applies; reg and
    greg need every wave to own one 64-block chunk (B <= 512)."""
    monkeypatch.setenv("WAL2026_DECODE_XMODE", mode)
    small, _g = _bench_layer([256], 1024, 2, 256, _lib.U8)
    rc, info = _info(small, 3)
    assert rc == _lib.OK and _lib.XMODE_NAMES[info.x_mode] == mode
    wide, _g2 = _bench_layer([256], 4608, 1, 4096, _lib.U16, 128)
    rc, info = _info(wide, 1)
    if mode in ("reg", "greg"):
        assert rc == _lib.EUNSUPPORTED and "WAL2026_DECODE_XMODE" in _lib.lib().wal_last_error().decode()
        # wal_rvq_linear refuses the same call before any launch
        rc2 = _lib.lib().wal_rvq_linear(ctypes.byref(wide), 0, 0, 0x8000000, 1, _lib.BF16, None, _lib.F32, 0x2000,
                                        _lib.BF16, None)
        assert rc2 == _lib.EUNSUPPORTED
    else:
        assert rc == _lib.OK and _lib.XMODE_NAMES[info.x_mode] == mode


def test_unknown_override_values_refused(monkeypatch):
    L, _g = _bench_layer([256], 1024, 2, 256, _lib.U8)
    monkeypatch.setenv("WAL2026_DECODE_XMODE", "fast")
    assert _info(L, 1)[0] == _lib.EINVAL
    monkeypatch.delenv("WAL2026_DECODE_XMODE")
    monkeypatch.setenv("WAL2026_PREFILL_TILE", "huge")
    assert _info(L, 64)[0] == _lib.EINVAL


def test_decode_falls_back_when_no_layout_fits(monkeypatch):
    """A one-stage table of 155,392 bytes (9712 entries) fits beside one
    tile's partial sums at M = 1 but not at M = 16 (8 waves x 16 x 16 fp32
    partials): there the call is routed to the generic kernel instead of
    failing at launch."""
    monkeypatch.delenv("WAL2026_DECODE_XMODE", raising=False)
    L, _g = _bench_layer([64], 128, 1, 9712, _lib.U16)
    assert _info(L, 1)[1].kernel == _lib.KERNEL_DECODE
    assert _info(L, 16)[1].kernel == _lib.KERNEL_GENERIC


def test_torch_operator_library_loads_and_refuses_cpu():
    """libwal2026_amd_torch.so registers torch.ops.wal2026_amd.rvq_linear over
    the C ABI; a CPU tensor is refused with RuntimeError (there is no CPU
    path), before the layer descriptor is touched."""
    import torch

    op = _lib.ops().rvq_linear
    with pytest.raises(RuntimeError, match="ROCm device"):
        op(torch.zeros(1, 64, dtype=torch.bfloat16), 0, 0, 0, None, None)
