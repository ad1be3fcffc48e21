"""Host-side brute force of the 16-bit implicit-GEMM convolution's index maps, through the library's own functions
(the ones its kernel and launcher call), with no GPU: for every batch from 1 to 64 and every convolution shape the
benchmark nets use, the launch covers each (pixel tile, column tile) exactly once, the column tiles of a pixel tile
share one XCD, and every convolution maps a 192-pixel region to the same XCD; and the direct loads that put a stage's
weights into LDS fill each stored chunk exactly once, with every wave issuing the same number of them (so that the
compiler's count of loads in flight is exact), and the swizzled fragment reads get back the logical chunks."""

import collections

import pytest

# (ks, ic, oc, split): the convolutions of b18c384nbt (stem 22 -> 384 3x3, bottleneck 384 -> 192 and 192 -> 384
# split 1x1, inner 192 -> 192 3x3, gpool 192 -> 256 3x3), b10c128 (128 -> 128 and the gpool 128 -> 160 3x3) and
# the 16-bit 1x1 on unsplit operands.
SHAPES = [(3, 22, 384, False), (3, 192, 192, False), (3, 192, 256, False), (3, 128, 128, False),
          (3, 128, 160, False), (1, 384, 192, True), (1, 192, 384, True), (1, 384, 192, False),
          (1, 192, 384, False)]
BATCHES = list(range(1, 65))


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[0]}_{s[1]}to{s[2]}{'_split' if s[3] else ''}")
def test_every_tile_is_computed_once_with_xcd_aware_order(kgx, shape):
    ks, ic, oc, split = shape
    for b in BATCHES:
        pixels = b * 361
        g = kgx.conv_geometry(ks, ic, oc, split, pixels)
        assert g["pixel_tiles"] == -(-pixels // g["tile_rows"]) and g["col_tiles"] == -(-oc // g["tile_cols"])
        seen = collections.Counter()
        xcd_of_tile = {}
        for wg in range(g["grid"]):
            mt, nt = kgx.conv_tile_of(ks, ic, oc, split, pixels, wg)
            if mt < 0:
                continue
            assert 0 <= mt < g["pixel_tiles"] and 0 <= nt < g["col_tiles"], (b, wg, mt, nt)
            seen[(mt, nt)] += 1
            # the column tiles of one pixel tile run on one XCD (workgroup id mod 8)
            assert xcd_of_tile.setdefault(mt, wg % 8) == wg % 8, (b, wg, mt)
            # and a 192-pixel region lands on the same XCD in every convolution (96-pixel tiles in pairs)
            region = mt * g["tile_rows"] // 192
            assert wg % 8 == region % 8, (b, wg, mt, g["tile_rows"])
        want = {(m, n) for m in range(g["pixel_tiles"]) for n in range(g["col_tiles"])}
        assert set(seen) == want and all(v == 1 for v in seen.values()), f"batch {b}: tiles missed or repeated"


@pytest.mark.parametrize("shape", [s for s in SHAPES if s[0] == 3], ids=lambda s: f"3x3_{s[1]}to{s[2]}")
def test_direct_weight_loads_fill_every_stored_chunk_once(kgx, shape):
    ks, ic, oc, split = shape
    g = kgx.conv_geometry(ks, ic, oc, split, 32 * 361)
    if not g["weights_direct"]:
        pytest.skip("this tile stages its weights through registers")
    rows = g["weight_rows"]
    assert g["direct_instructions"] * 8 == rows
    assert g["direct_per_wave"] == -(-g["direct_instructions"] // g["waves"])
    filled = collections.Counter()
    for w in range(g["waves"]):
        for q in range(g["direct_per_wave"]):  # every wave issues the same number of direct loads
            for lane in range(64):
                sr, sc, dr, dc = kgx.conv_weight_load(ks, ic, oc, split, q, w, lane)
                assert 0 <= sr < rows and 0 <= sc < 8, (w, q, lane, sr, sc)
                if dr < 0:  # a surplus load into the spare area: it still reads inside the tile's weights
                    continue
                assert sr == dr, (w, q, lane)
                # the lane stores chunk dc of row dr with the row's source chunk sc: the swizzle of dc
                assert sc == kgx.conv_weight_chunk(dr, dc)
                filled[(dr, dc)] += 1
    assert set(filled) == {(r, c) for r in range(rows) for c in range(8)}
    assert all(v == 1 for v in filled.values())
    # a fragment read of logical chunk c addresses stored chunk swizzle(c), which holds source chunk c
    for r in range(rows):
        for c in range(8):
            stored = kgx.conv_weight_chunk(r, c)
            assert kgx.conv_weight_chunk(r, stored) == c
        assert sorted(kgx.conv_weight_chunk(r, c) for c in range(8)) == list(range(8))


def test_geometry_rejects_bad_shapes(kgx):
    with pytest.raises(kgx.KgError, match="bad convolution shape"):
        kgx.conv_geometry(3, 192, 192, True, 361)  # split operands are 1x1 only
    with pytest.raises(kgx.KgError, match="workgroup out of range"):
        g = kgx.conv_geometry(3, 192, 192, False, 361)
        kgx.conv_tile_of(3, 192, 192, False, 361, g["grid"])
    with pytest.raises(kgx.KgError, match="through registers"):
        kgx.conv_weight_load(1, 384, 192, True, 0, 0, 0)


def test_junction_tiles_cover_every_pixel_once_on_the_convolutions_xcds(kgx):
    """The junction launch (a nested block's exit 1x1 and the next block's entry 1x1 in one kernel) over batches 1
    to 64: every 48-pixel tile exactly once, and each on the XCD (workgroup id mod 8) that the 192-pixel
    convolutions before and after it give its 192-pixel region."""
    for b in BATCHES:
        pixels = b * 361
        grid, _ = kgx.junction_tile_of(pixels, 0)
        seen = collections.Counter()
        for wg in range(grid):
            g, t = kgx.junction_tile_of(pixels, wg)
            assert g == grid
            if t < 0:
                continue
            assert 0 <= t * 48 < pixels, (b, wg, t)
            seen[t] += 1
            assert wg % 8 == (t * 48 // 192) % 8, (b, wg, t)
        assert set(seen) == set(range(-(-pixels // 48))) and all(v == 1 for v in seen.values()), b
        # the convolutions' 192-pixel tile of the same pixels runs on the same XCD
        g3 = kgx.conv_geometry(3, 192, 192, False, pixels)
        for wg in range(g3["grid"]):
            mt, _ = kgx.conv_tile_of(3, 192, 192, False, pixels, wg)
            if mt >= 0:
                assert wg % 8 == mt % 8
    with pytest.raises(kgx.KgError, match="workgroup out of range"):
        kgx.junction_tile_of(361, 10 ** 6)


@pytest.mark.parametrize("cg,cr", [(64, 192), (128, 128)])
def test_gpool_tiles_cover_every_tile_and_channel_once_on_the_convolutions_xcds(kgx, cg, cr):
    """The gpool blocks' tile launch over batches 1 to 64: every (192-pixel tile, channel share) pair exactly once,
    the shares partition the regular channels, and tile t runs on XCD t mod 8, where the convolutions before and
    after it (192-pixel tiles) run it."""
    for b in BATCHES:
        pixels = b * 361
        grid, _, _, share = kgx.gpool_tile_of(pixels, cg, cr, 0)
        assert cr % share == 0 and share % 8 == 0
        seen = collections.Counter()
        for wg in range(grid):
            g, t, c0, n = kgx.gpool_tile_of(pixels, cg, cr, wg)
            assert g == grid and n == share
            if t < 0:
                continue
            assert 0 <= t * 192 < pixels and 0 <= c0 < cr and c0 % share == 0, (b, wg, t, c0)
            assert wg % 8 == t % 8, (b, wg, t)
            seen[(t, c0)] += 1
        want = {(t, c) for t in range(-(-pixels // 192)) for c in range(0, cr, share)}
        assert set(seen) == want and all(v == 1 for v in seen.values()), b
    with pytest.raises(kgx.KgError, match="no tile share"):
        kgx.gpool_tile_of(361, 32, 96, 0)


@pytest.mark.parametrize("grid,threads", [(256, 512), (512, 256), (61 * 4, 512), (8 * 8 * 8, 256), (13, 64)])
def test_l2_touch_covers_each_line_once_per_xcd(kgx, grid, threads):
    """Each XCD's workgroups (g mod 8) touch lines 0 .. n x threads - 1 of the next op's weights once each."""
    for x in range(8):
        wgs = [g for g in range(x, grid, 8)]
        lines = collections.Counter(kgx.l2_touch_line(grid, g, t) for g in wgs for t in range(threads))
        assert set(lines) == set(range(len(wgs) * threads)) and all(v == 1 for v in lines.values()), (grid, x)


@pytest.mark.parametrize("channels", [384, 512, 768])
@pytest.mark.parametrize("region", [0, 64, 96, 128, 192, 40])
def test_rmsnorm_rows_cover_each_row_once_from_its_tile_xcd(kgx, channels, region):
    """The RMSNorm launch after a residual token GEMM: every token row is taken once, and (region > 0, a multiple
    of the rows per workgroup) a workgroup's rows lie in one row tile of `region` rows that was written on its own
    XCD (tile r on XCD r mod 8; workgroup g runs on XCD g mod 8). A region that is not whole workgroups (40) falls
    back to consecutive rows."""
    for batch in (1, 5, 32, 64):
        rows = batch * 361
        grid, _, _ = kgx.rmsnorm_rows_of(rows, channels, region, 0)
        seen = collections.Counter()
        for g in range(grid):
            _, first, count = kgx.rmsnorm_rows_of(rows, channels, region, g)
            for r in range(first, first + count):
                seen[r] += 1
            if count and region in (64, 96, 128, 192):
                assert (first // region) % 8 == g % 8 and (first + count - 1) // region == first // region, (g, first)
        assert set(seen) == set(range(rows)) and all(v == 1 for v in seen.values()), (channels, region, batch)
