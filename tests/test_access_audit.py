"""CPU audit of the gfx950 kernels' memory accesses (no GPU needed).

The index arithmetic of the GEMM (q4_gemm.hip) and the decode kernels
(q4_decode.hip) is restated here in numpy and checked against the buffers the host
allocates, for the benchmark's shapes and the awkward ones the GPU tests use:

* raw buffer loads: an in-range offset (below the resource's num_records) must read
  inside the real buffer, num_records never exceeds the buffer, and offsets meant to
  read zeros sit at or past num_records (the class of bug that once put a 2 GiB
  offset in range: a resource of 0xFFFFFFFF records made kOutOfRange valid);
* LDS reads and writes stay inside their arrays and the layout fits 160 KiB;
* every output tile, row block and split is visited exactly once, and stores stay
  inside y.

It restates the kernels' formulas rather than executing them, so a change to an
index expression in the .hip sources must be mirrored here."""

import numpy as np
import pytest

OOB = 0x80000000
LDS_BYTES = 160 * 1024


def chk_buf(name, off, size, num_records, real_bytes):
    off = np.asarray(off, dtype=np.int64)
    assert num_records <= real_bytes, (name, num_records, real_bytes)
    assert num_records <= 2 ** 31, (name, num_records)
    inr = off < num_records
    bad = inr & ((off < 0) | (off + size > num_records))
    assert not bad.any(), (name, off[bad][:5], num_records)


REC, REC_SB = 1152, 1024  # weight record bytes; its scale/bias words start 1 KiB in


def layout(n, k):
    g = k // 64
    nb = (n + 15) // 16
    gp = (g + 1) // 2
    # the kernels see the records as tiles (from the start) and as sb (REC_SB bytes in)
    return dict(n=n, k=k, g=g, nb=nb, gp=gp, rec_bytes=nb * gp * REC, sb_bytes=nb * gp * REC - REC_SB)


def sb_span(n):
    n = np.asarray(n, np.int64)
    return np.where(n > 0, n * REC - REC_SB, 0)


def in_tile_part(off, size):
    """Offsets from the record array's start that stay inside one record's tiled words."""
    off = np.asarray(off, np.int64)
    return ((off % REC) + size <= REC_SB).all()


def in_sb_part(off, size):
    """Offsets from the scale words' start (REC_SB in) that stay inside one record's words."""
    off = np.asarray(off, np.int64)
    return ((off % REC) + size <= REC - REC_SB).all()


# ------------------------------------------------------------------------- GEMM

def tile_of(bid, nwg, mtiles, ntiles):
    tile = bid
    if nwg % 8 == 0:
        tile = (bid % 8) * (nwg // 8) + bid // 8
    band = tile // (2 * ntiles)
    r = tile - band * 2 * ntiles
    bm = min(2, mtiles - band * 2)
    return band * 2 + r % bm, r // bm


def xprime_offset(c, k, kx):
    """Byte offset in x (rows of kx) of 16-byte unit c of x' (rows of k): column c of a
    two-plane handle's x' = [x | x] is column c mod kx of x."""
    c = np.asarray(c, np.int64)
    if kx == k:
        return c * 16
    row, cr = c // (k // 8), c % (k // 8)
    return (row * (kx // 8) + np.where(cr >= kx // 8, cr - kx // 8, cr)) * 16


def audit_gemm(m, n, k, BM, splits, BN=256, kx=None, q8=False):
    """kx: the row length of x (k, or k / 2 for a two-plane 8-bit handle).  q8: a
    two-plane handle in one pass (FORM 2): groups of K, the high plane's pair p and the
    low plane's pair G / 2 + p of each row block's records in one weight slot."""
    kx = kx or k
    L = layout(n, k)
    assert not q8 or (k == 2 * kx and (L["g"] // 2) % 2 == 0)
    WAVES = BN // 32   # side by side along N, each all BM rows x 32 columns
    RB = BN // 16
    MT = BM // 16                 # 16-row tiles per wave
    XP = BM * 8 // (64 * WAVES)   # x DMA parts per wave per group
    XIN = BM < 256 and not q8     # X_g summed in the kernel, else DMA'd from the pre-pass
    XT = (MT + WAVES - 1) // WAVES if XIN else 0  # row tiles whose X_g a wave sums: wave + WAVES t
    XA = 0 if XIN else MT // WAVES  # bias A-operand DMA parts per wave per octet
    SW = RB // 8                  # waves loading a pair's scale words
    assert RB == 2 * WAVES and XP >= 1 and (XT * WAVES >= MT if XIN else XA * WAVES == MT)
    # the DMAs issued from inside the product stream (after tile t of the wave's
    # (BM / 16) x 2 tiles): the x loads after tiles 1, 3, ..., the pair's weights after
    # tiles TW and TW + 2 -- every one must fall inside the stream or it is never issued
    TILES = MT * 2
    TW = 9 if TILES >= 12 else 5
    assert 2 * XP - 1 < TILES and TW + 2 < TILES, (BM, TILES, TW)
    KWP, KSP = RB * 64, RB * 16 // 2  # uint4 units of one plane's words, and of the scale words
    KWS = 2 * KWP if q8 else KWP      # a slot's words
    XAA = BM // 16 * 64               # uint4 units of the bias A operands
    BIAS_SLOT = XAA + RB * 4 * 16 // 2  # uint4 units: A operands, then the octet's scale/bias words
    G = L["g"] // 2 if q8 else L["g"]
    lo_pairs = G // 2 if q8 else 0
    octets = (G + 7) // 8
    mtiles = (m + BM - 1) // BM
    ntiles = (n + BN - 1) // BN
    nblocks = (n + 15) // 16
    xbytes = m * kx * 2
    gx = kx // 64
    ws_bytes = mtiles * (BM // 16) * octets * 1024  # the pre-pass's bias A operands
    per = (octets + splits - 1) // splits
    assert (octets + per - 1) // per == splits
    g_split = per * 8
    nwg = mtiles * ntiles
    seen = set()
    lane = np.arange(64)
    l16 = lane & 15
    for bid in range(nwg):
        mt, nt = tile_of(bid, nwg, mtiles, ntiles)
        assert 0 <= mt < mtiles and 0 <= nt < ntiles
        seen.add((mt, nt))
        # interior tiles repeat the first one's pattern shifted inside the buffers: the
        # edge tiles (first and last along M and N) bound every access
        if mt not in (0, mtiles - 1) and nt not in (0, ntiles - 1):
            continue
        rbw = nt * RB
        for wave in range(WAVES):
            # DMA offsets: per-lane constants + a scalar step offset (group, pair, octet)
            for part in range(XP):
                q = (WAVES * part + wave) * 64 + lane
                rr = q >> 3
                c = (q & 7) ^ ((rr >> 1) & 7)
                row = mt * BM + rr
                assert ((WAVES * part + wave) * 64 + 64) <= BM * 8
                xv = np.where(row < m, (row * kx + 8 * c) * 2, OOB)
                # a per-lane constant plus (g mod gx) * 128: the extremes bound every step
                for g in sorted({0, G - 1, min(G, gx) - 1, gx % G}):
                    gm = g - gx if g >= gx else g
                    assert 0 <= gm < gx
                    chk_buf("gemm x", np.where(xv == OOB, OOB, xv + gm * 128), 16, xbytes, xbytes)
            for part in range(2):
                rb = rbw + 2 * wave + part
                wv = np.where(rb < nblocks, rb * L["gp"] * REC + lane * 16, OOB)
                pairs = (0, G // 2 - 1, lo_pairs, lo_pairs + G // 2 - 1) if q8 else (0, L["gp"] - 1)
                for p in pairs:
                    off = np.where(wv == OOB, OOB, wv + p * REC)
                    chk_buf("gemm w", off, 16, L["rec_bytes"], L["rec_bytes"])
                    assert in_tile_part(off[off != OOB], 16)
            if wave < SW:
                rb = rbw + 8 * wave + (lane >> 3)
                sv = np.where(rb < nblocks, rb * L["gp"] * REC + (lane & 7) * 16, OOB)
                for p in (0, L["gp"] - 1):
                    off = np.where(sv == OOB, OOB, sv + p * REC)
                    chk_buf("gemm s", off, 16, L["sb_bytes"], L["sb_bytes"])
                    assert in_sb_part(off[off != OOB], 16)
            for o in sorted({0, octets - 1}):
                for u in range(XA):
                    m16 = XA * wave + u
                    assert m16 * 64 + 64 <= XAA
                    off = ((mt * (BM // 16) + m16) * octets + o) * 1024 + lane * 16
                    chk_buf("gemm xa", off, 16, ws_bytes, ws_bytes)
                rb = rbw + 2 * wave + (lane >> 5)
                chunk = lane & 31
                ok = (rb < nblocks) & (4 * o + (chunk >> 3) < (lo_pairs if q8 else L["gp"]))
                raw = (rb * L["gp"] + 4 * o + (chunk >> 3)) * REC + (chunk & 7) * 16
                chk_buf("gemm bias words", np.where(ok, raw, OOB), 16, L["sb_bytes"], L["sb_bytes"])
                assert in_sb_part(raw[ok], 16)
                assert XAA + wave * 64 + 63 < BIAS_SLOT  # the scale/bias part of the bias slot
            # LDS operand reads of the 16x16x32 product stream
            kq = lane >> 4
            for j in range(2):  # the wave's two row blocks
                rbl = wave * 2 + j
                assert rbl * 64 + 64 <= KWP and ((rbl * 16 + l16) < KSP * 2).all()
                assert KWP + rbl * 64 + 64 <= KWS or not q8  # the low plane's words
                assert ((((wave * 2 + j) * 4 + kq) * 16 + l16) < RB * 4 * 16).all()  # bias words, uint2
            for i in range(MT):  # the product stream's and the X_g sums' x fragments
                r = 16 * i + l16
                for c in (kq, 4 + kq):
                    idx = r * 8 + (c ^ ((r >> 1) & 7))
                    assert (idx >= 0).all() and (idx < BM * 8).all()
                assert i * 64 + 64 <= XAA  # bias A operands
            # the wave's bias A-operand writes: its row tiles wave + WAVES t
            for t in range(XT):
                if wave + WAVES * t < MT:
                    assert (wave + WAVES * t) * 64 + 64 <= XAA
            # stores: rows 4*kq + e of each 16-row tile, column l16 of the row block
            for i in range(MT):
                for e in range(4):
                    mrow = mt * BM + 16 * i + 4 * kq + e
                    assert (mrow < mtiles * BM).all()
    assert len(seen) == nwg
    # split-K: each split starts on an octet and the planes fit the partial buffer
    for sp in range(splits):
        gb = sp * g_split
        ge = min(G, gb + g_split)
        assert gb < ge and gb % 8 == 0
    # LDS: three x slots (two for one-pass 8-bit at 256 rows), two weight slots, the bias
    # slot; two 128 x 128 workgroups per CU
    xslots = 2 if (q8 and BM == 256) else 3
    lds = xslots * BM * 8 * 16 + 2 * (KWS + KSP) * 16 + BIAS_SLOT * 16
    assert lds <= (LDS_BYTES if BN == 256 else LDS_BYTES // 2)


GEMM_SHAPES = [(33, 40, 384), (300, 256, 640), (257, 130, 320), (64, 512, 3840), (512, 2048, 3840),
               (512, 3840, 4096), (2048, 15360, 3840), (2048, 3840, 15360), (33, 16, 64), (40, 48, 576),
               (300, 130, 1088), (256, 512, 3840), (2048, 8192, 3840), (2048, 3840, 8192)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("bm,bn", [(256, 256), (128, 256), (64, 256)])
def test_gemm_accesses(m, n, k, bm, bn):
    octets = (k // 64 + 7) // 8
    for s in sorted({1, 2, min(8, octets), octets}):
        per = (octets + s - 1) // s
        if (octets + per - 1) // per == s:
            audit_gemm(m, n, k, bm, s, bn)

# two-plane 8-bit handles: the tiled K' = 2K, x rows of K
@pytest.mark.parametrize("m,n,k", [(2048, 15360, 3840), (300, 130, 1088), (33, 48, 576), (64, 96, 3840)])
@pytest.mark.parametrize("bm,bn", [(256, 256), (128, 256), (64, 256)])
def test_gemm_accesses_two_plane(m, n, k, bm, bn):
    octets = (2 * k // 64 + 7) // 8
    for s in sorted({1, 2, min(8, octets), octets}):
        per = (octets + s - 1) // s
        if (octets + per - 1) // per == s:
            audit_gemm(m, n, 2 * k, bm, s, bn, kx=k)


# two-plane 8-bit handles in one pass (128- and 256-row tiles): groups of K, both
# planes' words
@pytest.mark.parametrize("m,n,k", [(2048, 15360, 3840), (300, 130, 1152), (33, 48, 256), (64, 96, 3840),
                                   (2048, 3840, 15360)])
@pytest.mark.parametrize("bm", [128, 256])
def test_gemm_accesses_one_pass_eight_bit(m, n, k, bm):
    octets = (k // 64 + 7) // 8
    for s in sorted({1, 2, min(8, octets), octets}):
        per = (octets + s - 1) // s
        if (octets + per - 1) // per == s:
            audit_gemm(m, n, 2 * k, bm, s, 256, kx=k, q8=True)


# ----------------------------------------------------------------------- decode

def _chunk_reads(first, n_in, rec_bytes, n_max=4):
    """A chunk's weight loads against resources over n_in records starting at record
    `first`: tiled words at lane*16 + i*REC (i < n_max) over n_in*REC bytes, and the
    scale words of pair i, row r at i*REC + 8r over sb_span(n_in) bytes from the first
    record's words.  Vectorized over chunks: pairs i < n_in must read inside their own
    record (and the buffer), pairs i >= n_in must fall outside the resource (zeros)."""
    first = np.asarray(first, np.int64)
    n_in = np.asarray(n_in, np.int64)
    assert (n_in >= 0).all()
    live = n_in > 0
    # resources end inside the records array
    assert ((first * REC + n_in * REC)[live] <= rec_bytes).all()
    assert ((first * REC + REC_SB + sb_span(n_in))[live] <= rec_bytes).all()
    assert (n_in * REC <= 2 ** 31).all()
    lane = np.arange(64)
    for i in range(n_max):
        toff = lane * 16 + i * REC
        soff = (lane & 15) * 8 + i * REC
        inside = i < n_in
        # in range exactly for the live pairs, and then within the tile / words part
        assert ((toff.max() + 16 <= n_in * REC) == inside).all() or not live.any()
        assert ((toff.min() >= n_in * REC) | inside).all()
        assert ((soff.max() + 8 <= sb_span(n_in)) == inside).all() or not live.any()
        assert ((soff.min() >= sb_span(n_in)) | inside).all()
        assert in_tile_part(toff, 16) and in_sb_part(soff, 8)


def audit_decode_stream(m_total, n, k, cus=256, kx=None):
    """decode_stream_kernel: persistent workgroups over row blocks, K split over waves,
    16-row slabs along grid y; x staged in LDS with zero padding and a -X table; x rows
    are kx long (k, or k / 2 for a two-plane handle's x' = [x | x])."""
    kx = kx or k
    L = layout(n, k)
    GPW = 4
    MT = 1 if m_total == 1 else 2 if m_total == 2 else 4 if m_total <= 4 else 16
    R = min(MT, 4)
    ms = min(m_total, 16)
    static_lds = 2 * 8 * R * 64 * 4
    lds_bytes = ms * (k + GPW * 128) * 2 + (L["gp"] + GPW) * 2 * 16 * 4
    stream_lds = lds_bytes + ms * 16
    if stream_lds + static_lds > LDS_BYTES:
        return False
    waves = min(8, (L["gp"] + GPW - 1) // GPW, L["gp"])
    per_cu = max(1, 20 // waves)
    per_cu = min(per_cu, LDS_BYTES // (stream_lds + static_lds))
    cap = cus * per_cu
    per_wg = (L["nb"] + cap - 1) // cap
    grid = (L["nb"] + per_wg - 1) // per_wg
    nbuf = 4 if per_cu == 1 and per_wg >= 16 else 2
    lane = np.arange(64)
    col, kq = lane & 15, lane >> 4
    bid = np.arange(grid)
    my_blocks = (L["nb"] - bid + grid - 1) // grid
    seen = np.zeros(L["nb"], np.int64)
    for wave in range(waves):
        gp0 = wave * L["gp"] // waves
        cnt = (wave + 1) * L["gp"] // waves - gp0
        assert cnt >= 1
        passes = (cnt + GPW - 1) // GPW
        # every chunk a workgroup's wave issues, nbuf past its last included (empty ranges)
        c = np.arange(int(my_blocks.max()) * passes + nbuf)
        B, C = np.meshgrid(bid, c, indexing="ij")
        chunks = (my_blocks * passes)[:, None]
        live = C < chunks
        rb = np.where(live, B + (C // passes) * grid, 0)
        assert (rb < L["nb"]).all()
        pas = C % passes
        n_in = np.where(live, np.minimum(cnt - pas * GPW, GPW), 0)
        _chunk_reads(rb * L["gp"] + gp0 + pas * GPW, n_in, L["rec_bytes"])
        if wave == 0:
            np.add.at(seen, rb[live & (pas == passes - 1)], 1)
    assert (seen == 1).all()
    for slab in range((m_total + 15) // 16):
        m_rows = min(16, m_total - 16 * slab)
        row16 = ((k + GPW * 128) >> 3) + 1
        negx_base = m_rows * row16
        tab = 2 * (L["gp"] + GPW) * 16
        assert negx_base * 16 + tab * 4 <= stream_lds
        arow = np.minimum(col, m_rows - 1)
        for wave in range(waves):
            gp0 = wave * L["gp"] // waves
            cnt = (wave + 1) * L["gp"] // waves - gp0
            for pas in range((cnt + GPW - 1) // GPW):
                gpb = gp0 + pas * GPW
                xp = arow * row16 + kq + gpb * 16
                for i in range(GPW):
                    for gi in range(2):
                        for h in (0, 4):
                            idx = xp + i * 16 + gi * 8 + h
                            assert (idx >= 0).all() and (idx < negx_base).all()
                        nidx = gpb * 32 + 4 * kq + i * 32 + gi * 16
                        assert (nidx + 4 <= tab).all()
        xchunks = (m_rows * k) >> 3
        rowc = k >> 3
        c = np.arange(xchunks)
        row = c // rowc
        cr = c - row * rowc
        assert (row * row16 + cr < negx_base).all() and ((cr >> 3) * 16 + row < tab).all()
        chk_buf("dec x", xprime_offset(c, k, kx), 16, m_rows * kx * 2, m_rows * kx * 2)
        pad = (GPW * 128) >> 3
        c = np.arange(m_rows * pad)
        assert ((c // pad) * row16 + rowc + (c % pad) < negx_base).all()
    return True


def audit_decode_rows(m, n, k, cus=256, GPW=4, NBUF=2, waves=4, per_cu=2):
    """decode_rows_kernel (M = 1): one wave per row block, NBUF chunks in flight."""
    L = layout(n, k)
    nb, gp = L["nb"], L["gp"]
    grid = min((nb + waves - 1) // waves, cus * per_cu)
    nw = grid * waves
    passes = (gp + GPW - 1) // GPW
    row16 = (k + GPW * 128) >> 3
    lds_bytes = m * (k + GPW * 128) * 2 + (gp + GPW) * 2 * 16 * 4
    assert lds_bytes <= LDS_BYTES
    negx_base = m * row16
    gw = np.arange(nw)
    my = np.where(gw < nb, (nb - gw + nw - 1) // nw, 0)
    c = np.arange(int(my.max()) * passes + NBUF)
    W, C = np.meshgrid(gw, c, indexing="ij")
    chunks = (my * passes)[:, None]
    live = C < chunks
    rb = np.where(live, W + (C // passes) * nw, 0)
    assert (rb < nb).all()
    gpb = (C % passes) * GPW
    n_in = np.where(live, np.minimum(GPW, gp - gpb), 0)
    _chunk_reads(rb * gp + gpb, n_in, L["rec_bytes"])
    seen = np.zeros(nb, np.int64)
    np.add.at(seen, rb[live & (C % passes == passes - 1)], 1)
    assert (seen == 1).all()
    kq = np.arange(64) >> 4
    for p in range(passes):
        gpb = p * GPW
        for i in range(GPW):
            for gi in range(2):
                idx = (m - 1) * row16 + kq + (gpb + i) * 16 + gi * 8 + 4
                assert (idx < negx_base).all()
                t = (gpb + i) * 32 + gi * 16 + 4 * kq + 3
                assert (t < 2 * (gp + GPW) * 16).all()


DECODE_SHAPES = [(40, 384), (64, 320), (16, 64), (4096, 3840), (2048, 3840), (3840, 4096), (15360, 3840),
                 (3840, 15360), (262144, 3840), (131072 + 48, 128), (33, 640), (70000, 3840), (76800 + 40, 3840)]


@pytest.mark.parametrize("n,k", DECODE_SHAPES)
@pytest.mark.parametrize("m", [1, 2, 4, 8, 9, 16, 17, 31])
def test_decode_stream_accesses(m, n, k):
    audit_decode_stream(m, n, k)


# two-plane 8-bit handles (K' = 2K, x rows of K)
@pytest.mark.parametrize("n,k", [(15360, 3840), (48, 576), (130, 1088), (4096, 3840), (262144, 3840)])
@pytest.mark.parametrize("m", [1, 2, 4, 8, 9, 16, 17, 31])
def test_decode_stream_accesses_two_plane(m, n, k):
    audit_decode_stream(m, n, 2 * k, kx=k)


@pytest.mark.parametrize("n,k", [(15360, 3840), (30720, 3840), (8192 + 48, 128), (8192, 640), (16 * 512, 3840)])
def test_decode_rows_accesses(n, k):
    audit_decode_rows(1, n, k)


def limb_config(nb, gp, cus=256):
    """q4_limbs.hip limb_config: (waves, workgroups per CU, chunks in flight, strided)."""
    nch = (gp + 1) // 2
    if nch >= 32 and nb <= cus:
        return 16, 1, 3, False
    if nb <= 4 * cus:
        return 8, 1, 2, False
    return 8, 3, 1, True


def audit_decode_limbs(n, k, kx=None, cus=256):
    """decode_limb_kernel (one row of x): per-workgroup row blocks, chunks of two
    records dealt to the waves in turn, x' limbs and the per-group table in LDS, the
    (row block, wave) slots, and the final stores."""
    kx = k if kx is None else kx
    L = layout(n, k)
    nb, gp = L["nb"], L["gp"]
    waves, per_cu, nbuf, strided = limb_config(nb, gp, cus)
    grid = min(nb, cus * per_cu)
    nch = (gp + 1) // 2
    stride = 784  # 4 groups x 3 limbs x 4 quarters x 16 B, then a zero unit
    nrb_max = (nb + grid - 1) // grid
    lds = nch * stride + nch * 4 * 8 + nrb_max * waves * 16 * 4
    assert lds <= LDS_BYTES
    lane = np.arange(64)
    col, quarter = lane & 15, lane >> 4
    sb_off = (quarter >> 1) * REC + REC_SB + col * 8 + (quarter & 1) * 4
    seen = np.zeros((nb, nch), np.int64)
    stored = np.zeros(nb, np.int64)
    for b in range(grid):
        if strided:
            rb0, nrb, rbs = b, (nb - b + grid - 1) // grid, grid
        else:
            rb0 = b * nb // grid
            nrb, rbs = (b * nb + nb) // grid - rb0, 1
        total = nrb * nch
        for w in range(waves):
            mine = (total - w + waves - 1) // waves if w < total else 0
            for i in range(mine + nbuf):  # the issues past the last chunk read nothing
                f = w + i * waves
                live = f < total
                i_rb, c = divmod(f, nch)
                left = gp - 2 * c
                nrec = min(2, left) if live else 0
                first = (rb0 + i_rb * rbs) * gp + 2 * c if live else 0
                base = first * REC
                for off, size in ((lane * 16, 16), (REC + lane * 16, 16), (sb_off, 4)):
                    inr = off < nrec * REC
                    assert (base + off[inr] + size <= L["rec_bytes"]).all()
                    assert (off[inr] + size <= nrec * REC).all()
                if live:
                    assert rb0 + i_rb * rbs < nb and i_rb < nrb
                    seen[rb0 + i_rb * rbs, c] += 1
                    # slot of (row block, wave) and the chunk's LDS operands
                    assert (i_rb * waves + w) * 16 + 15 < nrb * waves * 16
                    assert c * stride + 768 + 16 <= nch * stride
                    assert (c * 4 + 3) * 8 + 8 <= nch * 32
        for r in range(nrb):
            stored[rb0 + r * rbs] += 1
    assert (seen == 1).all() and (stored == 1).all()
    # staging: unit u of x' (u < nch * 32) -> limbs and table; x reads below kx * 2 bytes
    u = np.arange(nch * 32)
    g, h, kq = u >> 3, (u >> 2) & 1, u & 3
    base = (g >> 2) * stride + (g & 3) * 192 + kq * 16 + h * 8
    assert (base + 128 + 8 <= nch * stride).all() and ((base % stride) + 128 + 8 <= 768).all()
    assert (g * 8 + 8 <= nch * 32).all()
    xu = u[u < (k // 64) * 8]
    assert (xprime_offset(xu, k, kx) + 16 <= kx * 2).all()


@pytest.mark.parametrize("n,k", DECODE_SHAPES + [(8192, 3840), (1000, 192), (16, 128), (30720, 3840)])
def test_decode_limb_accesses(n, k):
    audit_decode_limbs(n, k)


@pytest.mark.parametrize("n,k", [(15360, 3840), (48, 576), (130, 1088), (3840, 15360), (262144, 3840)])
def test_decode_limb_accesses_two_plane(n, k):
    audit_decode_limbs(n, 2 * k, kx=k)


LIMB_BATCH = 2


def limb_rows_plan(nb, gp, mt, cus=256):
    """q4_limbs.hip limb_rows_plan: at 4 and 8 rows with more than 16 row blocks per CU
    one 16-wave workgroup per CU walking its run in phases of LIMB_BATCH row blocks (a
    two-phase ring of sums); else at 2 rows the one-row launch shape, at 4 and 8 the
    swept shapes; workgroups per CU capped by the LDS, then the grid doubled (up to one
    workgroup per row block) until one fits.  Returns (waves, nbuf, strided, grid, lds,
    batch)."""
    nch = (gp + 1) // 2
    if mt >= 4 and nb > 16 * cus:
        lds = nch * (4 * mt * 3 * 64 + 16) + nch * 4 * mt * 8 + 2 * LIMB_BATCH * 16 * mt * 16 * 4
        if lds <= LDS_BYTES:
            return 16, 2, True, cus, lds, LIMB_BATCH
    if mt == 2:
        waves, per_cu, nbuf, strided = limb_config(nb, gp, cus)
    elif nb <= 4 * cus:
        waves, per_cu, nbuf, strided = 16, 1, 2, False
    elif nb <= 16 * cus:
        waves, per_cu, nbuf, strided = 16, 2, 2 if mt == 8 else 1, True
    else:
        waves, per_cu, nbuf, strided = 8, 2, 2, True
    nch = (gp + 1) // 2

    def lds(g):
        nrb = (nb + g - 1) // g
        return nch * (4 * mt * 3 * 64 + 16) + nch * 4 * mt * 8 + nrb * waves * mt * 16 * 4

    while True:
        grid = min(nb, cus * per_cu)
        fit = LDS_BYTES // lds(grid)
        if fit >= per_cu or per_cu == 1:
            break
        per_cu = max(fit, 1)
    while lds(grid) > LDS_BYTES and grid < nb:
        grid = min(2 * grid, nb)
    return waves, nbuf, strided, grid, lds(grid), 0


def audit_decode_limb_rows(m_rows, n, k, kx=None, cus=256):
    """decode_limb_rows_kernel (2-8 rows of x): the chunk walk as in the one-row kernel;
    the scale-word loads; the staging of m_rows x' rows into [chunk][group][row][limb]
    [quarter] limb units, the (chunk, group, row) table and the zero unit; the A operand
    reads of every MFMA; the (row block, wave, row) slots and the final stores; with
    phases, the ring of slots (two row blocks live at once never share a slot) and each
    phase's stores."""
    kx = k if kx is None else kx
    mt = 2 if m_rows <= 2 else 4 if m_rows <= 4 else 8
    L = layout(n, k)
    nb, gp = L["nb"], L["gp"]
    waves, nbuf, strided, grid, lds, batch = limb_rows_plan(nb, gp, mt, cus)
    if lds > LDS_BYTES:
        return None  # the launcher refuses it (the bf16 kernels run)
    nch = (gp + 1) // 2
    chunk_bytes = 4 * mt * 3 * 64
    stride = chunk_bytes + 16
    lane = np.arange(64)
    col, quarter = lane & 15, lane >> 4
    sb0 = REC_SB + col * 8 + ((quarter >> 1) * 4 if mt == 2 else 0)
    sw_size = 4 if mt == 2 else 8
    seen = np.zeros((nb, nch), np.int64)
    stored = np.zeros((nb, mt), np.int64)
    nrb_max = 0
    for b in range(grid):
        if strided:
            rb0, nrb, rbs = b, (nb - b + grid - 1) // grid, grid
        else:
            rb0 = b * nb // grid
            nrb, rbs = (b * nb + nb) // grid - rb0, 1
        nrb_max = max(nrb_max, nrb)
        total = nrb * nch
        for w in range(waves):
            mine = (total - w + waves - 1) // waves if w < total else 0
            for i in range(mine + nbuf):
                f = w + i * waves
                live = f < total
                i_rb, c = divmod(f, nch)
                nrec = min(2, gp - 2 * c) if live else 0
                base = ((rb0 + i_rb * rbs) * gp + 2 * c) * REC if live else 0
                for off, size in ((lane * 16, 16), (REC + lane * 16, 16), (sb0, sw_size), (REC + sb0, sw_size)):
                    inr = off < nrec * REC
                    assert (off[inr] + size <= nrec * REC).all()
                    assert (base + off[inr] + size <= L["rec_bytes"]).all()
                if live:
                    seen[rb0 + i_rb * rbs, c] += 1
                    # the lane's slot rows (with phases: ring slot of the row block) and
                    # the chunk's table entries
                    srb = ((i_rb // batch) & 1) * batch + i_rb % batch if batch else i_rb
                    slot_rbs = 2 * batch if batch else nrb
                    assert ((srb * waves + w) * mt + mt - 1) * 16 + 15 < slot_rbs * waves * mt * 16
                    assert (c * 4 * mt + 3 * mt + mt - 1) < nch * 4 * mt
        if batch:
            # phase ph stores row blocks [ph batch, ph batch + batch) of the run from ring
            # half ph % 2; the row blocks of phases ph and ph + 1 (live together) take
            # different slots
            for ph in range((nrb + batch - 1) // batch):
                for r in range(batch):
                    if ph * batch + r < nrb:
                        stored[rb0 + (ph * batch + r) * rbs] += 1
            for i_rb in range(nrb):
                for j_rb in range(i_rb + 1, min(nrb, (i_rb // batch + 2) * batch)):
                    a = ((i_rb // batch) & 1) * batch + i_rb % batch
                    bb = ((j_rb // batch) & 1) * batch + j_rb % batch
                    assert a != bb, (i_rb, j_rb)
        else:
            for r in range(nrb):
                stored[rb0 + r * rbs] += 1
    assert (seen == 1).all() and (stored == 1).all()
    slot_rbs = 2 * batch if batch else nrb_max
    assert nch * stride + nch * 4 * mt * 8 + slot_rbs * waves * mt * 16 * 4 == lds
    # staging: flat unit f -> (row m, unit u); writes inside the chunk's limb region
    runits = nch * 32
    f = np.arange(mt * runits)
    m, u = f // runits, f % runits
    g, h, kq = u >> 3, (u >> 2) & 1, u & 3
    base = (g >> 2) * stride + (((g & 3) * mt + m) * 3) * 64 + kq * 16 + h * 8
    assert (base + 128 + 8 <= nch * stride).all() and ((base % stride) + 128 + 8 <= chunk_bytes).all()
    assert (((g >> 2) * 4 * mt + (g & 3) * mt + m) < nch * 4 * mt).all()
    ok = (m < m_rows) & (u < (k // 64) * 8)
    assert (m[ok] * kx * 2 + xprime_offset(u[ok], k, kx) + 16 <= m_rows * kx * 2).all()
    # every unit of a (row, group) lies in one 8-lane run (the max and sum shuffles)
    assert ((f // 8) == (m * runits + (u // 8) * 8) // 8).all()
    # A operands: MFMA i of a chunk, lane (row r = col, quarter)
    mfmas = 4 if mt <= 4 else 8
    gpa = 4 // mt if mt <= 4 else 1
    hits = np.zeros((4, mt, 3, 4), np.int64)
    for i in range(mfmas):
        for r in range(16):
            for q in range(4):
                l = r & 3
                if mt <= 4:
                    j, mm, on = i, (r % (4 * mt)) >> 2, (r // (4 * mt)) == (i % gpa) and l < 3
                else:
                    j, mm, on = i >> 1, 4 * (i & 1) + (r >> 2), l < 3
                off = ((j * mt + mm) * 3 + l) * 64 + q * 16 if on else chunk_bytes
                assert off + 16 <= stride
                if on:
                    hits[j, mm, l, q] += 1
    assert (hits == 1).all()  # every (group, row, limb, quarter) unit read by exactly one MFMA lane
    # final stores: t -> (row block run index, row, column) covers every output once
    # (with phases: t -> (row block of the phase, row, column) over a ring half)
    t = np.arange((batch if batch else nrb_max) * mt * 16)
    r, mm = t // (mt * 16), (t >> 4) % mt
    for half in ((0, batch) if batch else (0,)):
        assert ((((half + r) * waves + waves - 1) * mt + mm) * 16 + 15 < slot_rbs * waves * mt * 16).all()
    return lds


# the largest shapes (thousands of row blocks per launch) at 8 rows only, where the
# slots press hardest on the LDS
ROWS_SHAPES = [(40, 384), (64, 320), (16, 64), (4096, 3840), (2048, 3840), (3840, 4096), (15360, 3840),
               (3840, 15360), (33, 640), (8192, 3840), (40, 192), (1000, 192)]


@pytest.mark.parametrize("m", [2, 5, 8])
@pytest.mark.parametrize("n,k", ROWS_SHAPES)
def test_decode_limb_rows_accesses(m, n, k):
    audit_decode_limb_rows(m, n, k)


@pytest.mark.parametrize("n,k", [(30720, 3840), (262144, 3840), (70000, 3840), (131072 + 48, 128)])
def test_decode_limb_rows_accesses_wide(n, k):
    audit_decode_limb_rows(8, n, k)


@pytest.mark.parametrize("m", [2, 4, 8])
@pytest.mark.parametrize("n,k", [(15360, 3840), (48, 576), (3840, 15360)])
def test_decode_limb_rows_accesses_two_plane(m, n, k):
    audit_decode_limb_rows(m, n, 2 * k, kx=k)
