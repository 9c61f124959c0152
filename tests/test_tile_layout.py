"""CPU model of the GPU tile layout (heliopause_amd/csrc/hp_common.h).

Emulates, in numpy, the upload repack (repack.hip) and the reads and bit
unpacking of the matvec kernel (kquant_matvec.hip), then checks:
  * every 16-byte chunk slot of a weight is written exactly once and every
    kernel read stays inside the weight's byte range (so no launch reads out
    of bounds for the shapes the runner accepts);
  * the integers the kernel's unpack feeds to v_dot4 reproduce the oracle's
    exact aux32 / sumi for each block (the oracle is the reference's
    restatement, lib.rs:2116-2172 and 1923-1968).
"""
import numpy as np
import pytest

from heliopause_amd import synthetic as S

Q4K, Q6K = 1, 3


def choose_geometry(nb):
    for s in range(min(nb, 64), 0, -1):
        if nb % s:
            continue
        r = 64 // s
        if r * s >= 48 or s == 1:
            return dict(nb=nb, S=s, R=r, iters=nb // s)
    raise AssertionError


def tile_slots(rows, g, ch):
    """Yield (row, block, chunk, byte_offset, dplane_index) for every slot."""
    nb, s_, r_ = g["nb"], g["S"], g["R"]
    for t in range((rows + r_ - 1) // r_):
        row0 = t * r_
        rt = min(r_, rows - row0)
        lanes = rt * s_
        for it in range(g["iters"]):
            for k in range(lanes):
                row, block = row0 + k // s_, it * s_ + k % s_
                dpi = row0 * nb + it * lanes + k
                for c in range(ch):
                    off = (row0 * nb * ch + (it * ch + c) * lanes + k) * 16
                    yield row, block, c, off, dpi


def repack(type_id, raw, rows, k):
    nb = k // 256
    g = choose_geometry(nb)
    ch = 9 if type_id == Q4K else 13
    out = np.zeros(rows * nb * ch * 16, dtype=np.uint8)
    dplane = np.zeros(rows * nb, dtype=np.uint16)
    blocks = raw.reshape(rows, nb, -1)
    for row, block, c, off, dpi in tile_slots(rows, g, ch):
        b = blocks[row, block]
        if type_id == Q4K:
            if c == 0:
                out[off:off + 16] = b[0:16]
            else:
                qs = b[16:144]
                for e in range(4):
                    dw = 4 * (c - 1) + e
                    p, l = dw >> 3, dw & 7
                    out[off + 4 * e: off + 4 * e + 4] = [qs[32 * p + 8 * cc + l] for cc in range(4)]
        else:
            ql, qh, sc = b[0:128], b[128:192], b[192:208]
            if c < 8:
                for e in range(4):
                    dw = 4 * c + e
                    p, l = dw >> 3, dw & 7
                    h, sh = p >> 1, 4 * (p & 1)
                    for cc in range(4):
                        lo = (int(ql[64 * h + 8 * cc + l]) >> sh) & 15
                        hi = (int(ql[64 * h + 32 + 8 * cc + l]) >> sh) & 15
                        out[off + 4 * e + cc] = lo | (hi << 4)
            elif c < 12:
                for e in range(4):
                    dw = 4 * (c - 8) + e
                    q, l = dw >> 3, dw & 7
                    for cc in range(4):
                        out[off + 4 * e + cc] = qh[32 * q + 8 * cc + l] ^ 0xAA
            else:
                out[off:off + 16] = sc
            dplane[dpi] = int(b[208]) | (int(b[209]) << 8)
    return out, dplane, g


def dot4(a, b):
    av = np.frombuffer(np.uint32(a).tobytes(), dtype=np.int8).astype(np.int64)
    bv = np.frombuffer(np.uint32(b).tobytes(), dtype=np.int8).astype(np.int64)
    return int((av * bv).sum())


def q8_transposed(qs_block):
    """X[j][l] dwords: byte c = q8[32j + 8c + l] (q8k.hip output layout)."""
    x = np.zeros(64, dtype=np.uint32)
    for j in range(8):
        for l in range(8):
            byts = [np.uint8(np.int8(qs_block[32 * j + 8 * c + l])) for c in range(4)]
            x[8 * j + l] = int(byts[0]) | (int(byts[1]) << 8) | (int(byts[2]) << 16) | (int(byts[3]) << 24)
    return x


def kernel_ints(type_id, tiles, slot_off, lanes, x_t, bsums):
    """The matvec kernel's integer part for one lane (row, block)."""
    def chunk(c):
        o = slot_off + c * lanes * 16
        return np.frombuffer(tiles[o:o + 16].tobytes(), dtype=np.uint32)

    aux = [0] * 8
    if type_id == Q4K:
        c0 = chunk(0)
        s0, s1, s2 = int(c0[1]), int(c0[2]), int(c0[3])
        sc, mn = [0] * 8, [0] * 8
        for j in range(4):
            sc[j] = (s0 >> (8 * j)) & 63
            mn[j] = (s1 >> (8 * j)) & 63
            sc[j + 4] = ((s2 >> (8 * j)) & 15) | (((s0 >> (8 * j + 6)) & 3) << 4)
            mn[j + 4] = ((s2 >> (8 * j + 4)) & 15) | (((s1 >> (8 * j + 6)) & 3) << 4)
        sumi = sum(int(bsums[j]) * mn[j] for j in range(8))
        for p in range(4):
            for lq in range(2):
                D = chunk(1 + 2 * p + lq)
                for li in range(4):
                    d = int(D[li])
                    lo, hi = d & 0x0F0F0F0F, (d >> 4) & 0x0F0F0F0F
                    l = 4 * lq + li
                    aux[l] += sc[2 * p] * dot4(lo, x_t[8 * (2 * p) + l]) + sc[2 * p + 1] * dot4(hi, x_t[8 * (2 * p + 1) + l])
        return aux, sumi
    csc = chunk(12)
    sc = [int(np.int8(np.uint8((int(csc[g >> 2]) >> (8 * (g & 3))) & 255))) for g in range(16)]
    for j in range(8):
        for lq in range(2):
            Dl = chunk(2 * (j >> 1) + lq)
            Dh = chunk(8 + 2 * (j >> 2) + lq)
            for li in range(4):
                ql, qh = int(Dl[li]), int(Dh[li])
                nib = ((ql >> 2) & 0x3C3C3C3C) if (j & 1) else ((ql << 2) & 0x3C3C3C3C)
                u = j & 3
                w = (nib | ((qh << (6 - 2 * u)) & 0xC0C0C0C0)) & 0xFFFFFFFF
                l = 4 * lq + li
                xv = int(x_t[8 * j + l])
                aux[l] += sc[2 * j] * dot4(w & 0xFFFF, xv) + sc[2 * j + 1] * dot4(w & 0xFFFF0000, xv)
    return [a >> 2 for a in aux], 0


@pytest.mark.parametrize("type_id,rows,k", [(Q4K, 7, 2560), (Q4K, 13, 512), (Q6K, 7, 2560), (Q6K, 5, 10240),
                                            (Q4K, 3, 10240), (Q6K, 70, 256)])
def test_slots_cover_each_byte_once(type_id, rows, k):
    nb = k // 256
    g = choose_geometry(nb)
    ch = 9 if type_id == Q4K else 13
    total = rows * nb * ch * 16
    seen = np.zeros(rows * nb * ch, dtype=np.int32)
    dseen = np.zeros(rows * nb, dtype=np.int32)
    for row, block, c, off, dpi in tile_slots(rows, g, ch):
        assert 0 <= off and off + 16 <= total
        assert off % 16 == 0
        seen[off // 16] += 1
        if c == 0:
            dseen[dpi] += 1
    assert (seen == 1).all()
    assert (dseen == 1).all()
    # Q6_K: tiles + d plane = GGUF byte count
    if type_id == Q6K:
        assert total + 2 * rows * nb == rows * nb * 210
    else:
        assert total == rows * nb * 144


def test_geometry_lanes():
    for nb in range(1, 129):
        g = choose_geometry(nb)
        assert g["S"] * g["R"] <= 64 and g["S"] * g["iters"] == nb
        # chain lanes and LDS sizes used by the kernel stay bounded
        assert g["R"] * 9 * g["S"] <= 9 * 64


@pytest.mark.parametrize("type_id", [Q4K, Q6K])
def test_kernel_unpack_matches_oracle_ints(type_id, oracle):
    rows, k = 7, 512
    seed = S.derive(S.BASE_SEED, "layout", type_id)
    raw = S.q4_k_blocks(seed, rows, k) if type_id == Q4K else S.q6_k_blocks(seed, rows, k)
    x = S.activations(seed, 1, k)
    x[0, 3] = 0.0
    qs, d, bs = oracle.quantize_q8_k(x)
    tiles, dplane, g = repack(type_id, raw.reshape(-1), rows, k)
    nb = k // 256
    ch = 9 if type_id == Q4K else 13
    bb = 144 if type_id == Q4K else 210
    checked = 0
    for row, block, c, off, dpi in tile_slots(rows, g, ch):
        if c != 0:
            continue
        r_ = g["R"]
        row0 = (row // r_) * r_
        lanes = min(r_, rows - row0) * g["S"]
        xb = q8_transposed(qs[0, 256 * block: 256 * block + 256])
        aux, sumi = kernel_ints(type_id, tiles, off, lanes, xb, bs[0, 8 * block: 8 * block + 8])
        blk = raw[row, block * bb:(block + 1) * bb]
        ref_aux, ref_sumi = oracle.block_ints(type_id, blk, qs[0, 256 * block: 256 * block + 256],
                                              bs[0, 8 * block: 8 * block + 8])
        assert list(ref_aux) == aux, (row, block)
        assert ref_sumi == sumi
        if type_id == Q6K:
            assert dplane[dpi] == int(blk[208]) | (int(blk[209]) << 8)
        checked += 1
    assert checked == rows * nb
