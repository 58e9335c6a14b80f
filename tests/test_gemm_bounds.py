"""Every byte the GEMM kernels read or write through a scalar offset lies
inside its operand, for every tile, split and wave of the launches the
planner can make. The hardware range check of a buffer access covers only its
vector offset, so an access whose scalar offset (a K-step's slab, a row block)
runs past the operand would read or write whatever memory follows it; the
kernel must never form one. This restates, in integers, the offsets of
gemm.hip's a_loader (the consumers' A fragments), producer::load_w (the W
slab) and fixup's partial sums, with the step sequences of run_tile and
produce, and checks the largest byte each launch touches against the
operand's size; and that the persistent kernel's workgroups take every tile
once and request the next tile's first steps only after their own. (store_tile's stores and residual reads keep their whole
offset in the vector offset; test_gemm_gpu's ragged residual test covers
them.) CPU only."""
from __future__ import annotations

import itertools

import pytest

XGROUP_BYTES, XSUB_BYTES = 4096, 1024
TILE_ROWS, TILE_BYTES, TILE_MANT, TILE_K = 16, 1152, 1024, 64


def rows_pad(r):
    return (r + 255) // 256 * 256


def k_steps(k):
    return (k + 63) // 64


# (BM, BN, consumer waves) of cfg_big, cfg_small, cfg_glu and cfg_tiny
CONFIGS = [(256, 128, 4), (128, 128, 4), (256, 128, 8), (64, 64, 2)]


def consumer_steps(ns, last):
    """run_tile's A loads, as K-step indices from the tile's first step:
    steps 0 and 1 before the loop, steps k+2 and k+3 in each pair of the loop,
    each clamped to the operand's last step."""
    steps = [0, min(1, last)]
    k = 0
    while k + 1 < ns:
        steps += [min(k + 2, last), min(k + 3, last)]
        k += 2
    return steps


def producer_steps(ns, last):
    """produce()'s W loads: steps 0-3 in the prologue (clamped), k+4 and k+5
    in the steady state, then the guarded tail loads."""
    steps = [0, min(1, last), min(2, last), min(3, last)]
    k = 0
    while k + 5 < ns:
        steps += [k + 4, k + 5]
        k += 2
    while k < ns:
        if k + 2 < ns and k + 4 < ns:
            steps.append(k + 4)
        if k + 1 < ns and k + 3 < ns and k + 5 < ns:
            steps.append(k + 5)
        k += 2
    return steps


def producer_tail_requests(ns):
    """produce_tile's requests after its prologue, for a tile followed by
    another (`next`): ('own', step) for the tile's steps, ('next', step) for
    the next tile's first steps, in the order they are made."""
    req = [("own", 2), ("own", 3)]
    k = 0
    while k + 5 < ns:
        req += [("own", k + 4), ("own", k + 5)]
        k += 2
    while k < ns:
        if k + 2 < ns:
            if k + 4 < ns:
                req.append(("own", k + 4))
            elif k + 4 == ns:
                req.append(("next", 0))
        if k + 1 < ns and k + 3 < ns:
            if k + 5 < ns:
                req.append(("own", k + 5))
            elif k + 5 == ns + 1:
                req.append(("next", 1))
        k += 2
    return req


def persistent_tiles(T, G):
    """gemm_kernel_tiles' walk: workgroup b on XCD b % 8 takes the tiles of
    that XCD's run (xcd_order's contiguous run) from start + b // 8 in steps of
    G // 8."""
    g, out = G // 8, []
    for b in range(G):
        x = b % 8
        end = (x + 1) * (T // 8) + min(x + 1, T % 8)
        out.append(list(range(x * (T // 8) + min(x, T % 8) + b // 8, end, g)))
    return out


def check_launch(M, N, K, BM, BN, CWM, S, KG=1):
    nk = k_steps(K)
    Mp, Np = rows_pad(M), rows_pad(N)
    ks = Mp // 32 * XGROUP_BYTES             # p.a_kstride
    wks = Np // TILE_ROWS * TILE_BYTES       # W.w_kstride
    a_size, w_size = ks * nk, wks * nk       # the buffer resources' sizes
    WM, TI = BM // CWM, BM // CWM // 32
    mt, nt = (M + BM - 1) // BM, (N + BN - 1) // BN
    # the A fragment of the highest vector offset: wave's last 32-row group,
    # lane 63 (row 31, K-half 1), sub-step 3, 16 bytes
    a_vmax = lambda wm: (wm * WM // 32 + TI - 1) * XGROUP_BYTES + 31 * 32 + 16 + 3 * XSUB_BYTES + 16
    # the producer thread of the highest offset: tile BN/16-1, row 15, h 1, second 16 bytes
    w_vmax = (BN // 16 - 1) * TILE_BYTES + 15 * TILE_K + 32 + 16 + 16
    w_emax = (BN // 16 - 1) * TILE_BYTES + TILE_MANT + 15 * 8 + 4 + 4
    runs = []  # (split, K-group's first step, its steps)
    for split in range(S):
        k0 = split * nk // S
        ns = (split + 1) * nk // S - k0
        # run_tile: K-group g of the split takes the g-th of KG equal runs
        assert ns % KG == 0, (nk, S, KG)
        runs += [(split, k0 + g * (ns // KG), ns // KG) for g in range(KG)]
    for split, k0, ns in runs:
        last = nk - 1 - k0
        a_hi = max(consumer_steps(ns, last))
        w_hi = max(producer_steps(ns, last))
        assert k0 + a_hi <= nk - 1 and k0 + w_hi <= nk - 1, (M, N, K, BM, S, split)
        for tm in range(mt):
            m0 = tm * BM
            a0 = m0 // 32 * XGROUP_BYTES + k0 * ks
            for wm in range(CWM):
                assert a0 + a_hi * ks + a_vmax(wm) <= a_size, ("A", M, N, K, BM, S, split, tm, wm)
        for tn in range(nt):
            w0 = (tn * BN) // TILE_ROWS * TILE_BYTES + k0 * wks
            assert w0 + w_hi * wks + max(w_vmax, w_emax) <= w_size, ("W", M, N, K, BN, S, split, tn)
    if S > 1:
        # fixup: unit (u*T + t), wave, 1 KB pieces, all inside T*S*BM*BN*4
        T = mt * nt
        unit_bytes = BM * BN * 4
        top = ((S - 1) * T + T - 1) * unit_bytes + (CWM - 1) * WM * BN * 4 + WM * BN * 4
        assert top <= T * S * unit_bytes


SHAPES = [
    (1, 256, 64), (7, 200, 200), (100, 96, 8), (129, 1000, 520), (300, 200, 256), (600, 1000, 8192),
    (1024, 2560, 2560), (2048, 2560, 4096), (2048, 2560, 9728), (2048, 6144, 2560), (2048, 19456, 2560),
    (4096, 5120, 17408), (4096, 34816, 5120), (1536, 1024, 4096), (256, 4096, 1024),
    (1024, 1024, 1024), (1024, 3072, 1024), (1024, 1024, 4096), (65, 64, 64), (64, 65, 128),
]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_scalar_offsets_stay_inside_operands(M, N, K):
    nk = k_steps(K)
    for (BM, BN, CWM), S in itertools.product(CONFIGS, range(1, 17)):
        if S > 1 and nk // S < 4:
            continue  # the planner never splits below four steps a split
        check_launch(M, N, K, BM, BN, CWM, S)
    # 64x64 tiles as two K-groups (cfg_tiny2), in every split count the
    # launch accepts (nk a multiple of splits x groups)
    for S in range(1, 9):
        if nk % (2 * S) == 0 and nk // (2 * S) >= 1:
            check_launch(M, N, K, 64, 64, 2, S, KG=2)
    # the 128x160 tiles (cfg_o): unsplit, and only for weights of whole 160-row tiles
    if N % 160 == 0:
        check_launch(M, N, K, 128, 160, 4, 1)


def test_o_tiles_need_whole_160_row_weights():
    # the launch rule has teeth: 160-row tiles over a weight of 200 rows
    # would read rows its packed operand (256 rows) does not hold
    with pytest.raises(AssertionError):
        check_launch(1024, 200, 1024, 128, 160, 4, 1)


@pytest.mark.parametrize("ns", [4, 6, 8, 16, 40, 64, 152, 272])
def test_persistent_tile_requests_each_step_once(ns):
    # a tile followed by another requests each of its own steps 2..ns-1 once,
    # then the next tile's steps 0 and 1 into the registers that start it
    # (step 0 into the even set, step 1 into the odd one)
    req = producer_tail_requests(ns)
    own = [s for kind, s in req if kind == "own"]
    assert sorted(own) == list(range(2, ns))
    assert [s for kind, s in req if kind == "next"] == [0, 1]
    assert req.index(("next", 0)) > req.index(("own", ns - 2))
    assert req.index(("next", 1)) > req.index(("own", ns - 1))


@pytest.mark.parametrize("T,G", [(257, 256), (384, 256), (512, 256), (1216, 256), (768, 256), (300, 248), (1000, 8)])
def test_persistent_workgroups_cover_every_tile_once(T, G):
    walks = persistent_tiles(T, G)
    tiles = sorted(t for w in walks for t in w)
    assert tiles == list(range(T))
    assert all(len(w) >= 1 for w in walks)
    # the rounds stay balanced: no workgroup takes more than one tile more than another
    assert max(map(len, walks)) - min(map(len, walks)) <= 1


def test_unclamped_prefetch_would_leave_the_operand():
    # the check above has teeth: the step sequence without the clamp (the
    # kernel before it was added) reads past A's last step
    nk, ns, last = 40, 40, 39
    steps = [0, 1] + [s for k in range(0, ns - 1, 2) for s in (k + 2, k + 3)]
    assert max(steps) > last
    assert max(consumer_steps(ns, last)) == last



# (tile columns BN, wave columns WN, waves across) of the GLU launches
# (cfg_glu and cfg_small; cfg_tiny2)
GLU_CONFIGS = [(128, 128, 1), (64, 64, 1)]


@pytest.mark.parametrize("F", [32, 64, 96, 128, 160, 4096, 9728, 17408])
def test_glu_epilogue_columns_stay_inside_the_operand(F):
    # store_glu: the wave of tile column n0 holds h columns c0 = n0/2 + wn*HW
    # .. c0+HW-1, HW = WN/2. The launch's tiles cover the pair's 2F rows
    # rounded up to 128 (launch_any), so together they write every column of
    # the operand's padded width k_pad(F), its K padding included, each once,
    # and read only rows the packed pair holds (2F rounded up to 256)
    Fp = (F + 63) // 64 * 64
    rows_pad = (2 * F + 255) // 256 * 256
    for BN, WN, waves_n in GLU_CONFIGS:
        HW = WN // 2
        cols = []
        for n0 in range(0, (2 * F + 127) // 128 * 128, BN):
            assert n0 + BN <= rows_pad, (F, BN, n0)
            for wn in range(waves_n):
                c0 = n0 // 2 + wn * HW
                assert c0 + HW <= Fp, (F, BN, WN, n0, wn)
                cols += range(c0, c0 + HW)
        assert sorted(cols) == list(range(Fp)), (F, BN)


def test_glu_tiles_of_2f_alone_would_leave_padding_unwritten():
    # the rule has teeth: 64-column tiles over 2F = 192 rows alone write h
    # columns 0..95 of an operand 128 wide
    F, BN, HW = 96, 64, 32
    cols = [c for n0 in range(0, (2 * F + BN - 1) // BN * BN, BN) for c in range(n0 // 2, n0 // 2 + HW)]
    assert max(cols) + 1 < (F + 63) // 64 * 64


def band_rows(ld):
    """gemm.hip's band_rows: whole 256-row tiles of an output `ld` floats a
    row whose byte span stays under 2 GiB (0 if not even 256 rows fit)."""
    return (2 ** 31 - 1) // (ld * 4) // 256 * 256


@pytest.mark.parametrize("M,N,K", [(4096, 151936, 512), (4096, 151936, 2560), (8192, 262144, 5120),
                                   (3329, 160000, 64), (10000, 70000, 1024), (5000, 2097136, 256)])
def test_output_bands_stay_inside_operands(M, N, K):
    # A launch whose output span reaches 2 GiB runs as one launch a band of
    # rows (band_of): the band's activations start at its first row's 32-row
    # group (the K-step stride stays the whole operand's) and its output at
    # its first row. The bands cover every row once, each band's output span
    # is under 2 GiB, and every A fragment a band's tiles load lies inside
    # the whole expanded operand, for every tile shape.
    band = band_rows(N)
    assert band >= 256
    bands = [(r0, min(band, M - r0)) for r0 in range(0, M, band)]
    assert sum(rows for _, rows in bands) == M and bands[0][0] == 0
    assert all(r0 % 256 == 0 and rows * N * 4 < 2 ** 31 for r0, rows in bands)
    assert len(bands) > 1 or M * N * 4 < 2 ** 31
    nk = k_steps(K)
    ks = rows_pad(M) // 32 * XGROUP_BYTES
    a_size = ks * nk
    for r0, rows in bands:
        shift = r0 // 32 * XGROUP_BYTES
        for BM, _, CWM in CONFIGS:
            WM, TI = BM // CWM, BM // CWM // 32
            top = max((tm * BM // 32 + wm * WM // 32 + TI - 1) * XGROUP_BYTES
                      for tm in range((rows + BM - 1) // BM) for wm in range(CWM))
            a_hi = shift + top + 31 * 32 + 16 + 3 * XSUB_BYTES + 16 + (nk - 1) * ks
            assert a_hi <= a_size, (M, N, K, r0, rows, BM)


def producer_barriers(ns):
    """produce_tile's barriers for a tile of ns steps: one after the
    prologue, two per pair of the steady loop, then one per step of the
    tail."""
    n, k = 1, 0
    while k + 5 < ns:
        n += 2
        k += 2
    while k < ns:
        n += 1 + (1 if k + 1 < ns else 0)
        k += 2
    return n


def consumer_barriers(ns):
    """consume_tile's barriers: one before the first step, one per step."""
    n, k = 1, 0
    while k + 1 < ns:
        n += 2
        k += 2
    if k < ns:
        n += 1
    return n


@pytest.mark.parametrize("ns", [1, 2, 3, 4, 5, 6, 7, 8, 16, 32, 33, 64])
def test_every_wave_meets_the_same_barriers(ns):
    # a workgroup's waves meet each s_barrier together: a tile's producers and
    # consumers meet ns + 1, and with K-groups every group runs the same ns
    # (the launch requires nk to be a multiple of splits x groups) and every
    # wave meets one more, where groups 1.. hand their sums to group 0
    assert producer_barriers(ns) == consumer_barriers(ns) == ns + 1


def kgroup_lds(BM, BN, KG, waves, WM, WN):
    """run_tile's LDS map of a K-group launch: (rings, sums regions, group
    0's epilogue regions, LDS_BYTES), each a list of [lo, hi) byte ranges."""
    ring = 3 * BN * 128
    tile = BM * BN * 4
    lds = KG * max(ring, tile)
    rings = [(g * ring, (g + 1) * ring) for g in range(KG)]
    sums = [(g * tile + w * WM * WN * 4, g * tile + (w + 1) * WM * WN * 4) for g in range(1, KG) for w in range(waves)]
    epilogue = [(w * WM * WN * 4, (w + 1) * WM * WN * 4) for w in range(waves)]
    return rings, sums, epilogue, lds


@pytest.mark.parametrize("KG", [2, 3, 4])
def test_kgroup_lds_regions(KG):
    # cfg_tiny2's map (64x64 tiles, two consumer waves of 32x64), and the
    # same tiles with three or four groups: every region inside the
    # workgroup's LDS, the rings apart, the sums apart from each other and
    # from group 0's epilogue regions (which the residual DMA, the GLU
    # staging and the split-K fixup use while group 0 finishes)
    rings, sums, epi, lds = kgroup_lds(64, 64, KG, 2, 32, 64)
    regions = rings + sums + epi
    assert all(0 <= lo < hi <= lds for lo, hi in regions)
    assert lds <= 160 * 1024
    def apart(rs):
        rs = sorted(rs)
        return all(a[1] <= b[0] for a, b in zip(rs, rs[1:]))
    assert apart(rings) and apart(sums + epi)
