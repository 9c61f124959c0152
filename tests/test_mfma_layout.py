"""CPU model of the matrix-core kernels' weight operands (kquant_mfma.hip,
kquant_prefill.hip).

The kernels' A fragments are defined on a 16-row "segment" image of each
(16 rows, block): `repack_mfma` below writes it from the GGUF blocks, and
`emulate` runs the decode kernel's arithmetic on it (lane layout of
v_mfma_f32_16x16x32_f16: A lane i holds row i%16, k = 8*(i//16)..+7; B lane
i holds column i%16, the same k; D lane i holds rows 4*(i//16)+j, column
i%16; the f32 tail in block order).  By default the segment image is also
the second resident copy the kernels read; a weight kept in one layout
(hp_hip_set_weight_layouts(0)) stays resident only in the vector-ALU tile
layout (test_tile_layout.repack), and each kernel gathers its lanes' dwords
from there with tile_row's offsets.  Checks:
  * the segment image holds every byte once, the weight's byte count per
    16-row tile;
  * the emulated MFMA accumulators equal the oracle's exact per-lane-class
    integers (aux32, sumi: lib.rs:2116-2172, 1923-1968) and stay below 2^24,
    where f16 x f16 products summed in f32 are exact, and the outputs equal
    the oracle's matmul bit for bit;
  * what each kernel's loads take from the tile layout -- the decode
    kernel's lane registers, the bit-exact prefill kernel's LDS image, the
    fast prefill kernel's fragment dwords -- equals the segment image, and
    every load stays inside the weight's tiles, for one- and two-iteration
    geometries and ragged row counts.
"""
import numpy as np
import pytest

from heliopause_amd import synthetic as S

Q4K, Q6K = 1, 3
SEG = {Q4K: 2304, Q6K: 3360}


def elem(j, c, l):
    """Element index of (sub-block j, position c, lane class l): 32j + 8c + l."""
    return 32 * j + 8 * c + l


def q4k_fields(blk):
    s = blk[4:16].astype(np.int64)
    sc, mn = [], []
    for j in range(8):
        if j < 4:
            sc.append(s[j] & 63)
            mn.append(s[j + 4] & 63)
        else:
            sc.append((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4))
            mn.append((s[j + 4] >> 4) | ((s[j] >> 6) << 4))
    e = np.arange(256)
    q = (blk[16 + 32 * (e // 64) + e % 32] >> (4 * ((e // 32) % 2))) & 15
    return np.array(sc), np.array(mn), q.astype(np.int64)


def q6k_fields(blk):
    e = np.arange(256)
    h, t, l = e // 128, (e % 128) // 32, e % 32
    lo = (blk[64 * h + l + 32 * (t & 1)] >> (4 * (t >> 1))) & 15
    hi = (blk[128 + 32 * h + l] >> (2 * t)) & 3
    return (lo | (hi << 4)).astype(np.int64), blk[192:208].view(np.int8).astype(np.int64)


def repack_mfma(type_id, raw, rows, k):
    """Tile segments: (tile T, block b) at (b * tiles + T) * SEG (block-major).
    Q4_K: [0,256) 16 row headers (GGUF bytes 0..15); [256, 2304) chunk c in
      {0,1} x lane i (row i%16, quarter q = i//16): 16 bytes = dwords u = 0..3
      of class l = 2q + c, byte cc of dword u = q(2u, cc, l) | q(2u+1, cc, l) << 4.
    Q6_K: [0,256) 16 rows x 16 int8 scales; [256,288) 16 f16 d; [288, 3360)
      chunk c in {0,1,2} x lane i: c < 2 as Q4_K with the low 4 bits of q6;
      c = 2: dword 2*cls + h holds, in byte cc, the high 2 bits of q6 at
      (j = 4h + jj, cc, class 2q + cls) in bits 2jj.
    Rows past the weight in the last tile are zero."""
    nb = k // 256
    tiles = (rows + 15) // 16
    out = np.zeros(tiles * nb * SEG[type_id], dtype=np.uint8)
    written = np.zeros_like(out, dtype=np.int32)
    blocks = raw.reshape(rows, nb, -1)
    for T in range(tiles):
        for b in range(nb):
            base = (b * tiles + T) * SEG[type_id]
            for rho in range(16):
                r = T * 16 + rho
                blk = blocks[r, b] if r < rows else None
                if type_id == Q4K:
                    hdr = blk[0:16] if blk is not None else np.zeros(16, np.uint8)
                    out[base + 16 * rho: base + 16 * rho + 16] = hdr
                    written[base + 16 * rho: base + 16 * rho + 16] += 1
                    _, _, q = q4k_fields(blk) if blk is not None else (None, None, np.zeros(256, np.int64))
                    for qq in range(4):
                        i = qq * 16 + rho
                        for c in range(2):
                            l = 2 * qq + c
                            for u in range(4):
                                for cc in range(4):
                                    v = q[elem(2 * u, cc, l)] | (q[elem(2 * u + 1, cc, l)] << 4)
                                    off = base + 256 + (c * 64 + i) * 16 + 4 * u + cc
                                    out[off] = v
                                    written[off] += 1
                else:
                    if blk is not None:
                        q6, sc = q6k_fields(blk)
                        out[base + 16 * rho: base + 16 * rho + 16] = blk[192:208]
                        out[base + 256 + 2 * rho: base + 258 + 2 * rho] = blk[208:210]
                    else:
                        q6 = np.zeros(256, np.int64)
                    written[base + 16 * rho: base + 16 * rho + 16] += 1
                    written[base + 256 + 2 * rho: base + 258 + 2 * rho] += 1
                    for qq in range(4):
                        i = qq * 16 + rho
                        for c in range(2):
                            l = 2 * qq + c
                            for u in range(4):
                                for cc in range(4):
                                    v = (q6[elem(2 * u, cc, l)] & 15) | ((q6[elem(2 * u + 1, cc, l)] & 15) << 4)
                                    off = base + 288 + (c * 64 + i) * 16 + 4 * u + cc
                                    out[off] = v
                                    written[off] += 1
                        for cls in range(2):
                            l = 2 * qq + cls
                            for h in range(2):
                                for cc in range(4):
                                    v = 0
                                    for jj in range(4):
                                        v |= (q6[elem(4 * h + jj, cc, l)] >> 4) << (2 * jj)
                                    off = base + 288 + (2 * 64 + i) * 16 + 4 * (2 * h + cls) + cc
                                    out[off] = v
                                    written[off] += 1
    return out, written


def lane_a_fragment(type_id, seg, i, g, u):
    """f16 values (exact ints) lane i supplies as A of MFMA (group g, u):
    class 2q+g, elements (j = 2u, c = 0..3) then (j = 2u+1, c = 0..3), each
    times its group scale."""
    rho, q = i % 16, i // 16
    if type_id == Q4K:
        hdr = seg[16 * rho: 16 * rho + 16]
        blk = np.concatenate([hdr, np.zeros(128, np.uint8)])
        sc, _, _ = q4k_fields(blk)
        dw = seg[256 + (g * 64 + i) * 16 + 4 * u: 256 + (g * 64 + i) * 16 + 4 * u + 4]
        lo = [int(x) & 15 for x in dw]
        hi = [int(x) >> 4 for x in dw]
        return [sc[2 * u] * v for v in lo] + [sc[2 * u + 1] * v for v in hi]
    sc = seg[16 * rho: 16 * rho + 16].view(np.int8).astype(np.int64)
    dw = seg[288 + (g * 64 + i) * 16 + 4 * u: 288 + (g * 64 + i) * 16 + 4 * u + 4]
    h = u // 2
    qh = seg[288 + (2 * 64 + i) * 16 + 4 * (2 * h + g): 288 + (2 * 64 + i) * 16 + 4 * (2 * h + g) + 4]
    vals = []
    for half, j in ((0, 2 * u), (1, 2 * u + 1)):
        jj = j - 4 * h
        for cc in range(4):
            lo = (int(dw[cc]) >> (4 * half)) & 15
            hi = (int(qh[cc]) >> (2 * jj)) & 3
            grp = 2 * j + (cc >= 2)
            vals.append(int(sc[grp]) * ((lo | (hi << 4)) - 32))
    return vals


def q8k(x):
    from oracle import oracle as O
    return O.quantize_q8_k(x)


def emulate(type_id, seg_bytes, rows, k, x):
    """Runs the kernel's arithmetic for all tiles; returns [M][rows] f32."""
    nb = k // 256
    m_cols = x.shape[0]
    qs, dx, _ = q8k(x)
    qs = qs.reshape(m_cols, nb, 256).astype(np.int64)
    out = np.zeros((m_cols, rows), np.float32)
    tiles = (rows + 15) // 16
    nset = (m_cols + 3) // 4
    for T in range(tiles):
        sums = np.zeros((nset, 64, 2, 4), np.float32)   # [set][lane][g][j]
        sumf = np.zeros((nset, 64, 4), np.float32)
        for b in range(nb):
            base = (b * tiles + T) * SEG[type_id]
            seg = seg_bytes[base: base + SEG[type_id]]
            for st in range(nset):
                acc = np.zeros((2, 16, 16), np.int64)   # [g][row][n]
                for g in range(2):
                    for u in range(4):
                        A = np.zeros((16, 32), np.int64)
                        B = np.zeros((32, 16), np.int64)
                        for i in range(64):
                            a = lane_a_fragment(type_id, seg, i, g, u)
                            A[i % 16, 8 * (i // 16): 8 * (i // 16) + 8] = a
                            n, qq = i % 16, i // 16
                            m, s = 4 * st + n % 4, n // 4
                            if m < m_cols and qq == s:
                                l = 2 * qq + g
                                xs = [qs[m, b, elem(2 * u + (e >= 4), e % 4, l)] for e in range(8)]
                                B[8 * qq: 8 * qq + 8, n] = xs
                        assert np.abs(A).max() <= 2048 and np.abs(B).max() <= 2048  # exact in f16
                        acc[g] += A @ B
                        assert np.abs(acc[g]).max() < 2 ** 24
                if type_id == Q4K:
                    A = np.zeros((16, 32), np.int64)
                    B = np.zeros((32, 16), np.int64)
                    _, _, bs16 = bsums16(qs[:, b])
                    for i in range(64):
                        rho, qq = i % 16, i // 16
                        if qq < 2:
                            hdr = seg[16 * rho: 16 * rho + 16]
                            _, mn, _ = q4k_fields(np.concatenate([hdr, np.zeros(128, np.uint8)]))
                            A[rho, 8 * qq: 8 * qq + 8] = [mn[4 * qq + e // 2] for e in range(8)]
                            n = i % 16
                            m = 4 * st + n % 4
                            if n < 4 and m < m_cols:
                                B[8 * qq: 8 * qq + 8, n] = bs16[m, 8 * qq: 8 * qq + 8]
                    accmin = A @ B
                # tail: lane i holds rows 4*(i//16)+j, column n = i % 16
                for i in range(64):
                    n = i % 16
                    m, s = 4 * st + n % 4, n // 4
                    if m >= m_cols:
                        continue
                    for j in range(4):
                        rho = 4 * (i // 16) + j
                        r = T * 16 + rho
                        if r >= rows:
                            continue
                        if type_id == Q4K:
                            dw = np.frombuffer(seg[16 * rho: 16 * rho + 2].tobytes(), np.float16)[0]
                            dmw = np.frombuffer(seg[16 * rho + 2: 16 * rho + 4].tobytes(), np.float16)[0]
                        else:
                            dw = np.frombuffer(seg[256 + 2 * rho: 258 + 2 * rho].tobytes(), np.float16)[0]
                        dd = np.float32(np.float32(dw) * dx[m, b])
                        for g in range(2):
                            p = np.float32(dd * np.float32(acc[g][rho, n]))
                            sums[st, i, g, j] = np.float32(sums[st, i, g, j] + p)
                        if type_id == Q4K and s == 0:
                            dm = np.float32(np.float32(dmw) * dx[m, b])
                            sumf[st, i, j] = np.float32(sumf[st, i, j] - np.float32(dm * np.float32(accmin[rho, n])))
        # final: s_l for class l = 2s + g lives in lane n = m%4 + 4s (row group), group g
        for st in range(nset):
            for m4 in range(4):
                m = 4 * st + m4
                if m >= m_cols:
                    continue
                for rho in range(16):
                    r = T * 16 + rho
                    if r >= rows:
                        continue
                    grp, j = rho // 4, rho % 4
                    tot = np.float32(-0.0)
                    for l in range(8):
                        s, g = l // 2, l % 2
                        tot = np.float32(tot + sums[st, 16 * grp + m4 + 4 * s, g, j])
                    if type_id == Q4K:
                        tot = np.float32(sumf[st, 16 * grp + m4, j] + tot)
                    out[m, r] = tot
    return out


def bsums16(qs_b):
    """Per column, sums of the 16 elements lane 2j+u of the Q8_K prologue
    owns (32j + 8c + 4u + i, c, i = 0..3): halves of each bsums32."""
    m_cols = qs_b.shape[0]
    bs = np.zeros((m_cols, 16), np.int64)
    for j in range(8):
        for u in range(2):
            idx = [32 * j + 8 * c + 4 * u + i for c in range(4) for i in range(4)]
            bs[:, 2 * j + u] = qs_b[:, idx].sum(axis=1)
    assert np.abs(bs).max() <= 2048
    return None, None, bs


@pytest.mark.parametrize("type_id", [Q4K, Q6K])
def test_repack_writes_each_byte_once(type_id):
    rows, k = 21, 512
    raw = (S.q4_k_blocks if type_id == Q4K else S.q6_k_blocks)(3, rows, k)
    out, written = repack_mfma(type_id, raw, rows, k)
    assert (written == 1).all()
    assert out.size == ((rows + 15) // 16) * (k // 256) * SEG[type_id]
    assert SEG[type_id] == 16 * (144 if type_id == Q4K else 210)


@pytest.mark.parametrize("type_id,rows,m_cols", [(Q4K, 18, 1), (Q4K, 16, 6), (Q6K, 19, 3), (Q6K, 16, 5)])
def test_emulated_kernel_matches_oracle(oracle, type_id, rows, m_cols):
    k = 512
    raw = (S.q4_k_blocks if type_id == Q4K else S.q6_k_blocks)(rows + m_cols, rows, k)
    x = S.activations(type_id * 100 + rows, m_cols, k)
    x[0, 7] = -50.0
    segs, _ = repack_mfma(type_id, raw, rows, k)
    got = emulate(type_id, segs, rows, k, x)
    want = oracle.matmul(type_id, raw, x, rows).reshape(m_cols, rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q6k_f16_operand_exactness_criterion():
    """The matrix-core kernels take sc * (q - 32) as an f16 operand.  The set of
    int8 scales for which some 6-bit quant makes that product inexact in f16
    is exactly the odd scales with |sc| >= 67 -- the condition the Q6_K repack
    flags (those weights then run the vector-ALU kernels).  Checked over every
    (scale, quant) pair."""
    sc = np.arange(-128, 128, dtype=np.int64)[:, None]
    qq = np.arange(-32, 32, dtype=np.int64)[None, :]
    prod = sc * qq
    inexact = (prod.astype(np.float16).astype(np.int64) != prod).any(axis=1)
    flagged = (sc[:, 0] % 2 != 0) & (np.abs(sc[:, 0]) >= 67)
    assert np.array_equal(inexact, flagged)
    # the synthetic distribution (scales -32..31) never reaches it
    assert not inexact[(sc[:, 0] >= -32) & (sc[:, 0] <= 31)].any()


# ---- gathers from the tile layout -----------------------------------------

from test_tile_layout import repack as tile_repack  # noqa: E402


def tile_row(row, rows, g, ch):
    """hp_common.h tile_row: (base, chunk, iter, dbase, diter)."""
    nb, s_, r_ = g["nb"], g["S"], g["R"]
    t = row // r_
    r, row0 = row - t * r_, t * r_
    rt = min(r_, rows - row0)
    chunk = rt * s_ * 16
    return dict(base=(row0 * nb * ch + r * s_) * 16, chunk=chunk, iter=ch * chunk,
                dbase=row0 * nb + r * s_, diter=rt * s_)


def tile_off(tr, b, g, c):
    i, s = divmod(b, g["S"])
    return tr["base"] + i * tr["iter"] + c * tr["chunk"] + 16 * s


def _take(buf, off, n):
    assert 0 <= off and off + n <= buf.size, (off, n, buf.size)
    return buf[off:off + n]


def _dwords(b):
    return [int(x) for x in np.frombuffer(b.tobytes(), np.uint32)]


def _seg(segs, type_id, rows, nb, T, b):
    tiles = (rows + 15) // 16
    base = (b * tiles + T) * SEG[type_id]
    return segs[base: base + SEG[type_id]]


SHAPES = [(Q4K, 21, 512), (Q4K, 37, 10240), (Q6K, 19, 512), (Q6K, 40, 10240), (Q4K, 16, 2560),
          (Q6K, 7, 2560)]


def _weights(type_id, rows, k):
    raw = (S.q4_k_blocks if type_id == Q4K else S.q6_k_blocks)(rows + 7, rows, k)
    tiles_b, dplane, g = tile_repack(type_id, raw, rows, k)
    segs, _ = repack_mfma(type_id, raw, rows, k)
    return tiles_b, dplane, g, segs


@pytest.mark.parametrize("type_id,rows,k", SHAPES)
def test_decode_kernel_tile_loads(type_id, rows, k):
    """kquant_mfma.hip load_seg: lane i = (rho, q) of segment T, block b."""
    tiles_b, dplane, g, segs = _weights(type_id, rows, k)
    nb, ch = k // 256, (9 if type_id == Q4K else 13)
    for T in range((rows + 15) // 16):
        for i in range(64):
            rho, q = i % 16, i // 16
            row = min(16 * T + rho, rows - 1)
            tr = tile_row(row, rows, g, ch)
            oq = ((1 if type_id == Q4K else 0) + (q >> 1)) * tr["chunk"] + 8 * (q & 1)
            for b in range(nb):
                off = tile_off(tr, b, g, 0)
                p = [_dwords(_take(tiles_b, off + oq + 2 * u * tr["chunk"], 8)) for u in range(4)]
                c0 = [p[u][0] for u in range(4)]
                c1 = [p[u][1] for u in range(4)]
                seg = _seg(segs, type_id, rows, nb, T, b)
                if 16 * T + rho >= rows:
                    continue  # a re-read of the last row; its sums are never stored
                base = 256 if type_id == Q4K else 288
                assert c0 == _dwords(seg[base + 16 * i: base + 16 * i + 16])
                assert c1 == _dwords(seg[base + 1024 + 16 * i: base + 1024 + 16 * i + 16])
                if type_id == Q4K:
                    assert np.array_equal(_take(tiles_b, off, 16), seg[16 * rho: 16 * rho + 16])
                else:
                    assert np.array_equal(_take(tiles_b, off + 12 * tr["chunk"], 16), seg[16 * rho: 16 * rho + 16])
                    ib, sb = divmod(b, g["S"])
                    di = tr["dbase"] + ib * tr["diter"] + sb
                    assert 0 <= di < dplane.size
                    assert int(dplane[di]) == int(np.frombuffer(seg[256 + 2 * rho: 258 + 2 * rho].tobytes(), np.uint16)[0])
                    h0 = _dwords(_take(tiles_b, off + oq + 8 * tr["chunk"], 8))
                    h1 = _dwords(_take(tiles_b, off + oq + 10 * tr["chunk"], 8))
                    c2 = [v ^ 0xAAAAAAAA for v in h0 + h1]
                    assert c2 == _dwords(seg[2336 + 16 * i: 2336 + 16 * i + 16])


@pytest.mark.parametrize("type_id,rows,k", SHAPES)
def test_bit_exact_prefill_stage(type_id, rows, k):
    """kquant_prefill.hip stage_load + stage_store: the 32-row tile's LDS
    image equals its two segments (live rows)."""
    tiles_b, dplane, g, segs = _weights(type_id, rows, k)
    nb, ch = k // 256, (9 if type_id == Q4K else 13)
    segb = SEG[type_id]
    nseg = (rows + 15) // 16
    for T0 in range(0, nseg, 2):
        for b in range(nb):
            img = np.zeros(2 * segb, np.uint8)
            for tid in range(256):
                tr = tile_row(min(16 * T0 + (tid & 31), rows - 1), rows, g, ch)
                for r in range(2):
                    u = tid + 256 * r
                    if u >= 32 * ch:
                        continue
                    c, rl = u >> 5, u & 31
                    rho = rl & 15
                    w = _dwords(_take(tiles_b, tile_off(tr, b, g, c), 16))
                    sb = (rl >> 4) * segb
                    if c == (0 if type_id == Q4K else 12):
                        img[sb + 16 * rho: sb + 16 * rho + 16] = np.array(w, np.uint32).view(np.uint8)
                    elif type_id == Q4K or c < 8:
                        ck = c - 1 if type_id == Q4K else c
                        for e in range(4):
                            l = 4 * (ck & 1) + e
                            o = sb + (256 if type_id == Q4K else 288) + 1024 * (l & 1) + 16 * (16 * (l >> 1) + rho) + 4 * (ck >> 1)
                            img[o: o + 4] = np.array([w[e]], np.uint32).view(np.uint8)
                    else:
                        ck = c - 8
                        for e in range(4):
                            l = 4 * (ck & 1) + e
                            o = sb + 2336 + 16 * (16 * (l >> 1) + rho) + 4 * (2 * (ck >> 1) + (l & 1))
                            img[o: o + 4] = np.array([w[e] ^ 0xAAAAAAAA], np.uint32).view(np.uint8)
                if type_id == Q6K and tid < 32:
                    ib, s_ = divmod(b, g["S"])
                    di = tr["dbase"] + ib * tr["diter"] + s_
                    o = (tid >> 4) * segb + 256 + 2 * (tid & 15)
                    img[o: o + 2] = np.array([dplane[di]], np.uint16).view(np.uint8)
            for rs in range(2):
                if T0 + rs >= nseg:
                    continue
                seg = _seg(segs, type_id, rows, nb, T0 + rs, b)
                got = img[rs * segb: (rs + 1) * segb]
                for rho in range(16):
                    if 16 * (T0 + rs) + rho >= rows:
                        continue
                    # every byte of row rho: header/scales, d, and its units
                    idx = list(range(16 * rho, 16 * rho + 16))
                    if type_id == Q6K:
                        idx += [256 + 2 * rho, 257 + 2 * rho]
                    base = 256 if type_id == Q4K else 288
                    nun = 2 if type_id == Q4K else 3
                    for cidx in range(nun):
                        for qq in range(4):
                            o = base + 1024 * cidx + 16 * (16 * qq + rho)
                            idx += list(range(o, o + 16))
                    assert np.array_equal(got[idx], seg[idx])


@pytest.mark.parametrize("type_id,rows,k", SHAPES)
def test_fast_prefill_fragment_dwords(type_id, rows, k):
    """kquant_prefill.hip f3_wload: lane (n, q)'s dwords of class l = 2t + g
    (dword l % 4 of its chunk l / 4) are dword q of segment unit (l / 2, n) of
    chunk l % 2; Q6_K high bits likewise; scales and d of row n."""
    tiles_b, dplane, g, segs = _weights(type_id, rows, k)
    nb, ch = k // 256, (9 if type_id == Q4K else 13)
    for T in range((rows + 15) // 16):
        for n in range(16):
            if 16 * T + n >= rows:
                continue
            for q in range(4):
                tr = tile_row(min(16 * T + n, rows - 1), rows, g, ch)
                oq = (1 + 2 * q if type_id == Q4K else 2 * q) * tr["chunk"]
                oh = (8 + 2 * (q >> 1)) * tr["chunk"]
                for b in range(nb):
                    off = tile_off(tr, b, g, 0)
                    qa = [_dwords(_take(tiles_b, off + oq + x * tr["chunk"], 16)) for x in range(2)]
                    seg = _seg(segs, type_id, rows, nb, T, b)
                    base = 256 if type_id == Q4K else 288
                    for l in range(8):
                        t, gg = l >> 1, l & 1
                        unit = base + 1024 * gg + 16 * (16 * t + n)
                        assert qa[l >> 2][l & 3] == _dwords(seg[unit: unit + 16])[q]
                    if type_id == Q4K:
                        assert np.array_equal(_take(tiles_b, off, 16), seg[16 * n: 16 * n + 16])
                    else:
                        qh = [_dwords(_take(tiles_b, off + oh + x * tr["chunk"], 16)) for x in range(2)]
                        for t in range(4):
                            unit = _dwords(seg[2336 + 16 * (16 * t + n): 2336 + 16 * (16 * t + n) + 16])
                            for gg in range(2):
                                got = qh[t >> 1][2 * (t & 1) + gg] ^ 0xAAAAAAAA
                                assert got == unit[2 * (q >> 1) + gg]
                        gs = _dwords(_take(tiles_b, off + 12 * tr["chunk"] + 4 * q, 4))[0]
                        assert gs == _dwords(seg[16 * n + 4 * q: 16 * n + 4 * q + 4])[0]
                        ib, s_ = divmod(b, g["S"])
                        di = tr["dbase"] + ib * tr["diter"] + s_
                        assert int(dplane[di]) == int(np.frombuffer(seg[256 + 2 * n: 258 + 2 * n].tobytes(), np.uint16)[0])
