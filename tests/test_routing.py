"""Which kernel serves a call: the library's routing (plan_call in
csrc/qmm.hip, exposed by i4_plan_query) pinned for a table of shapes, so a
routing change shows here and not only as time.  CPU only: the plan is made
from the shape alone.

Routes: "decode" (dec_kernel, row groups of up to four), "decode8"
(dec8_kernel, row groups of eight), "prefill" (the INT8-MFMA GEMM), "rows"
(the rows kernel: block-integer export, legacy corr past the decode rows),
None (no single launch takes a paired or multi-projection call; the library
then runs the projections one by one).  Quantizer: None when the decode
prologue quantizes the activation, else the stand-alone one launched first.
"""
import pytest

# (bits, M, K, N, call flags) -> expected plan fields.
TABLE = [
    # The benchmark configurations.
    ("C1 W8 GEMV", (8, 1, 4096, 4096, {}), dict(route="decode", quant=None, p64=1, tile_ranges=256, grid_x=256)),
    ("C2 W4 GEMV", (4, 1, 4096, 12288, {}), dict(route="decode", quant=None, p64=1, tile_ranges=256)),
    ("C3 1 row", (4, 1, 12288, 4096, {}), dict(route="decode", quant=None, p64=1)),
    ("C3 2 rows", (4, 2, 12288, 4096, {}), dict(route="decode", quant=None, p64=1, row_groups=1)),
    ("C3 3 rows", (4, 3, 12288, 4096, {}), dict(route="decode", quant="staged", p64=0, row_groups=1)),
    ("C3 4 rows", (4, 4, 12288, 4096, {}), dict(route="decode", quant="staged", p64=0, rows_per_group=4,
                                                 row_groups=1)),
    ("C3 8 rows", (4, 8, 12288, 4096, {}), dict(route="decode8", quant="rows8", row_groups=1, lrec=0)),
    ("C4 W8 prefill", (8, 512, 5120, 17408, {}), dict(route="prefill", quant="prefill", pf_rp=4, pf_ct=17,
                                                      grid_x=64, grid_y=4)),
    ("C5 LM head", (8, 1, 5120, 151936, dict(argmax=True)), dict(route="decode", quant=None, p64=1)),
    # The prefill shape at other row counts.
    ("W4 prefill", (4, 512, 5120, 17408, {}), dict(route="prefill", pf_rp=4, pf_ct=17)),
    ("W8 16 rows", (8, 16, 5120, 17408, {}), dict(route="decode8", row_groups=2, tile_ranges=128, pair_xcd=1,
                                                   lrec=1)),
    ("W8 128 rows", (8, 128, 5120, 17408, {}), dict(route="prefill", pf_rp=4, pf_ct=5)),
    ("W8 LM head 9 rows", (8, 9, 5120, 151936, dict(argmax=True)), dict(route="prefill", pf_rp=1)),
    ("W8 LM head 8 rows", (8, 8, 5120, 151936, dict(argmax=True)), dict(route="decode8")),
    # Decode row limits by width.
    ("W4 256 tiles 32 rows", (4, 32, 12288, 4096, {}), dict(route="decode8", row_groups=4)),
    ("W4 256 tiles 33 rows", (4, 33, 12288, 4096, {}), dict(route="prefill")),
    ("W8 1088 tiles 17 rows", (8, 17, 5120, 17408, {}), dict(route="prefill")),
    # Where the four-row groups quantize in their prologue (K <= 4096).
    ("W8 K=N=4096 8 rows", (8, 8, 4096, 4096, {}), dict(route="decode", quant=None, row_groups=2, pair_xcd=1)),
    ("W8 K=4096 N=12288 8 rows", (8, 8, 4096, 12288, {}), dict(route="decode8", quant="rows8")),
    ("W4 K=4096 N=4096 12 rows", (4, 12, 4096, 4096, {}), dict(route="decode8")),
    ("W4 K=2048 N=8192 12 rows", (4, 12, 2048, 8192, {}), dict(route="decode", quant=None, row_groups=3)),
    ("W4 K=2048 N=8192 24 rows", (4, 24, 2048, 8192, {}), dict(route="decode8", row_groups=3)),
    # Long K: fewer rows per row group on the four-row groups.
    ("W4 K=26624 2 rows", (4, 2, 26624, 5120, {}), dict(route="decode", quant="staged", rows_per_group=1,
                                                        row_groups=2)),
    ("W4 K=17408 3 rows", (4, 3, 17408, 5120, {}), dict(route="decode", quant="staged", rows_per_group=2,
                                                        row_groups=2)),
    # Tall-skinny: few column tiles over a long K.
    ("W4 K=17408 N=64", (4, 1, 17408, 64, {}), dict(route="decode", quant=None, tile_ranges=4, grid_x=4,
                                                     split=0)),
    # Split-K: at most 8 tiles with at least 20 phases (15 chunks) a tile,
    # S workgroups a tile filling the CUs, at most one phase each.
    ("split W8 K=24576 N=64", (8, 1, 24576, 64, {}), dict(route="decode", quant=None, split=26, grid_x=104,
                                                           tile_ranges=4, row_groups=1)),
    ("split W8 K=32768 N=128 2 rows", (8, 2, 32768, 128, {}), dict(route="decode", quant=None, p64=1, split=32,
                                                                   grid_x=256)),
    ("split W4 K=40960 N=64", (4, 1, 40960, 64, {}), dict(route="decode", quant=None, split=22, grid_x=88)),
    ("split W8 K=18432 N=16 4 rows", (8, 4, 18432, 16, {}), dict(route="decode", quant=None, p64=0, split=20,
                                                                 rows_per_group=4, row_groups=1)),
    ("no split: 19 phases", (8, 1, 17408, 64, {}), dict(split=0, grid_x=4)),
    ("no split: 9 tiles", (8, 1, 32768, 144, {}), dict(split=0)),
    ("no split: fold staging past LDS", (8, 4, 20480, 16, {}), dict(split=0)),
    ("no split: argmax", (8, 1, 32768, 64, dict(argmax=True)), dict(split=0)),
    ("no split: 5 rows", (8, 5, 32768, 64, {}), dict(split=0)),
    # Non-temporal weight loads: plain decode calls whose tiles leave at most
    # one in eight producer slots idle.
    ("stream C3 1 row", (4, 1, 12288, 4096, {}), dict(route="decode", stream=1)),
    ("stream C3 4 rows", (4, 4, 12288, 4096, {}), dict(route="decode", quant="staged", stream=1)),
    ("stream C5 (argmax)", (8, 1, 5120, 151936, dict(argmax=True)), dict(route="decode", stream=1)),
    ("stream W4 K=5120", (4, 1, 5120, 17408, {}), dict(stream=1)),
    ("no stream C1: 11 of 75 slots idle", (8, 1, 4096, 4096, {}), dict(stream=0)),
    ("stream: gate/up pair with phases across tiles", (4, 1, 5120, 17408, dict(pair=True)), dict(flow=1, stream=1)),
    ("no stream: gate/up pair on the eight-row groups", (4, 20, 5120, 17408, dict(pair=True)),
     dict(route="decode8", flow=0, stream=0)),
    ("no stream: split-K", (8, 1, 24576, 64, {}), dict(split=26, stream=0)),
    # Phases across tile boundaries: several tiles a workgroup, whole chunks
    # that do not fill whole phases; then one stream of chunks leaves few
    # slots idle, so those calls read non-temporally too.
    ("flow C2", (4, 1, 4096, 12288, {}), dict(route="decode", flow=1, stream=1)),
    ("flow C5", (8, 1, 5120, 151936, dict(argmax=True)), dict(route="decode", flow=1, stream=1)),
    ("no flow C1: one tile a workgroup", (8, 1, 4096, 4096, {}), dict(flow=0, stream=0)),
    ("no flow C3: one tile a workgroup", (4, 1, 12288, 4096, {}), dict(flow=0, stream=1)),
    ("no flow: 30 chunks a tile fill whole phases", (4, 1, 3840, 12288, {}), dict(flow=0)),
    ("no flow: padded last chunk", (4, 1, 4064, 12288, {}), dict(flow=0)),
    ("flow: gate/up pair (gate and up tiles alternate)", (4, 1, 4096, 4096, dict(pair=True)), dict(flow=1)),
    ("no flow: multi-projection", (4, 1, 5120, 10240, dict(multi=True)), dict(flow=0, stream=0)),
    ("stream C3 8 rows (eight-row groups, one row group)", (4, 8, 12288, 4096, {}),
     dict(route="decode8", row_groups=1, stream=1)),
    ("stream W8 16 rows (two row groups)", (8, 16, 5120, 17408, {}), dict(route="decode8", row_groups=2, stream=1)),
    ("no stream: three row groups", (4, 24, 12288, 4096, {}), dict(route="decode8", row_groups=3, stream=0)),
    ("W4 K=17408 N=64 2 rows", (4, 2, 17408, 64, {}), dict(route="decode", quant="staged")),
    ("W4 K=24576 1 row", (4, 1, 24576, 4096, {}), dict(route="decode", quant=None)),
    ("W4 K=25600 1 row", (4, 1, 25600, 4096, {}), dict(route="decode", quant="staged")),
    # The export of block integers, and a legacy corr past the decode rows.
    ("block dots", (4, 4, 1024, 256, dict(dots=True)), dict(route="rows", quant="staged", grid_x=16, grid_y=1)),
    ("legacy corr 40 rows", (8, 40, 1024, 256, dict(legacy_corr=True)), dict(route="rows", grid_y=5)),
    ("legacy corr 16 rows", (8, 16, 1024, 256, dict(legacy_corr=True)), dict(route="decode", row_groups=4)),
    # Fused decoder calls.
    ("gate/up 1 row", (4, 1, 5120, 17408, dict(pair=True)), dict(route="decode", quant=None)),
    ("gate/up 20 rows", (4, 20, 5120, 17408, dict(pair=True)), dict(route="decode8", row_groups=3, lrec=1)),
    ("gate/up 20 rows K=4096", (4, 20, 4096, 4096, dict(pair=True)), dict(route=None)),
    ("multi 1 row", (4, 1, 5120, 10240, dict(multi=True)), dict(route="decode", quant=None)),
    ("multi with argmax", (4, 1, 5120, 10240, dict(multi=True, argmax=True)), dict(route=None)),
    ("multi with explicit zero points", (4, 1, 5120, 10240, dict(multi=True, extra=True)), dict(route=None)),
    ("norm + multi 2 rows", (4, 2, 5120, 10240, dict(multi=True, norm=True)), dict(route="decode", quant=None)),
    ("norm + multi 3 rows", (4, 3, 5120, 10240, dict(multi=True, norm=True)), dict(route=None)),
]


@pytest.mark.parametrize("name,call,want", TABLE, ids=[t[0] for t in TABLE])
def test_route(hb, name, call, want):
    bits, M, K, N, kw = call
    got = hb.plan(bits, M, K, N, n_cu=256, **kw)
    assert {k: got[k] for k in want} == want, got


def test_overrides_steer_the_route(hb, monkeypatch):
    assert hb.plan(4, 8, 12288, 4096)["route"] == "decode8"
    monkeypatch.setenv("BREEZE_HIP_DEC8", "0")
    p = hb.plan(4, 8, 12288, 4096)
    assert (p["route"], p["row_groups"]) == ("decode", 2)
    monkeypatch.setenv("BREEZE_HIP_DEC8", "2")
    assert hb.plan(8, 8, 4096, 4096)["route"] == "decode8"
    monkeypatch.delenv("BREEZE_HIP_DEC8")
    monkeypatch.setenv("BREEZE_HIP_DEC_ROWS", "4")
    assert hb.plan(4, 5, 4096, 4096)["route"] == "rows"  # past the decode rows, under the GEMM's 9
    assert hb.plan(4, 9, 4096, 4096)["route"] == "prefill"


def test_split_overrides(hb, monkeypatch):
    """BREEZE_HIP_SPLIT: 0 never, 1 wherever it fits, n >= 2 forces n pieces
    (at most one a phase)."""
    assert hb.plan(8, 1, 24576, 64)["split"] == 26
    monkeypatch.setenv("BREEZE_HIP_SPLIT", "0")
    assert hb.plan(8, 1, 24576, 64)["split"] == 0
    monkeypatch.setenv("BREEZE_HIP_SPLIT", "1")
    assert hb.plan(4, 1, 17408, 64)["split"] == 10  # 10 phases, 4 tiles
    assert hb.plan(4, 1, 4096, 1024)["split"] == 3  # 64 tiles: 256 / 64 = 4 pieces, 3 phases
    assert hb.plan(4, 1, 4096, 4096)["split"] == 0  # one workgroup a tile already fills the CUs
    assert hb.plan(4, 1, 1024, 64)["split"] == 0  # one phase a tile
    monkeypatch.setenv("BREEZE_HIP_SPLIT", "3")
    p = hb.plan(4, 1, 17408, 64)
    assert (p["split"], p["grid_x"]) == (3, 12)
    monkeypatch.setenv("BREEZE_HIP_SPLIT", "64")
    assert hb.plan(4, 1, 17408, 64)["split"] == 10


def test_stream_override(hb, monkeypatch):
    """BREEZE_HIP_STREAM: 0 / 1 turn non-temporal weight loads off / on for
    every plain decode call and gate/up pairs with phases across tiles
    (never multi-projection calls or split-K)."""
    assert hb.plan(8, 1, 5120, 151936, argmax=True)["stream"] == 1
    monkeypatch.setenv("BREEZE_HIP_STREAM", "0")
    assert hb.plan(8, 1, 5120, 151936, argmax=True)["stream"] == 0
    monkeypatch.setenv("BREEZE_HIP_STREAM", "1")
    assert hb.plan(8, 1, 4096, 4096)["stream"] == 1
    assert hb.plan(4, 1, 5120, 17408, pair=True)["stream"] == 1  # a pair with phases across tiles
    monkeypatch.setenv("BREEZE_HIP_FLOW", "0")
    assert hb.plan(4, 1, 5120, 17408, pair=True)["stream"] == 0  # a pair without
    assert hb.plan(4, 1, 5120, 10240, multi=True)["stream"] == 0


def test_flow_override(hb, monkeypatch):
    """BREEZE_HIP_FLOW: 0 / 1 turn phases across tile boundaries off / on
    wherever they apply (tiles of at least 15 whole chunks, plain calls)."""
    assert hb.plan(4, 1, 4096, 12288)["flow"] == 1
    monkeypatch.setenv("BREEZE_HIP_FLOW", "0")
    assert hb.plan(4, 1, 4096, 12288)["flow"] == 0
    monkeypatch.setenv("BREEZE_HIP_FLOW", "1")
    assert hb.plan(8, 1, 4096, 4096)["flow"] == 1  # one tile a workgroup: same phases
    assert hb.plan(4, 1, 1024, 12288)["flow"] == 0  # 8 chunks a tile
    assert hb.plan(4, 1, 4064, 12288)["flow"] == 0  # padded last chunk
    assert hb.plan(4, 1, 5120, 17408, multi=True)["flow"] == 0


def test_plan_follows_the_device_size(hb):
    """Tile ranges and row groups come from the compute-unit count."""
    assert hb.plan(4, 1, 4096, 12288, n_cu=304)["tile_ranges"] == 304
    p = hb.plan(4, 16, 12288, 4096, n_cu=128)
    assert (p["row_groups"], p["tile_ranges"]) == (2, 64)


def test_plan_query_rejects_bad_arguments(hb):
    with pytest.raises(ValueError):
        hb.plan(4, 0, 4096, 4096)
    with pytest.raises(ValueError):
        hb.plan(4, 1, 4095, 4096)
