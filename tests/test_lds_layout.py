"""Address identities the attention kernels rely on (autoresearch_amd/csrc/ar_flash.hip).

K / V / Q / dO tiles sit in LDS as natural rows of HD bf16 values whose 16-byte
chunks are XOR-swizzled per row (Geo::off).  The MFMA fragment reads do not
recompute that swizzle per read:

* rowfrag_x: the fragment of k-step ks for row lane % 32 of 32-row block kb is
  at kb * 32 * HD elements + (rowbase(lane) ^ (ks * 32)) bytes;
* trfrag_x: the two 8-byte transposed reads of (rb, s, ct) are at
  (32 rb + 16 s) * HD elements + (tb{0,1}(lane) ^ (64 ct)) bytes.

Both are checked here exhaustively against the swizzled layout for every lane,
block and k-step at the head dims the kernels are built for.
"""
import pytest


def geo(hd):
    nch = hd // 8

    def swz(r):
        return (4 * (r & 3) + ((r >> 2) & 3)) & (nch - 1)

    def off(r, c):  # element offset of logical (row, chunk)
        return r * hd + ((c ^ swz(r)) << 3)

    return off


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_row_fragment_xor(hd):
    off = geo(hd)
    ksteps = hd // 16
    for lane in range(64):
        base = 2 * off(lane & 31, lane >> 5)
        for kb in range(2):
            for ks in range(ksteps):
                direct = 2 * off(kb * 32 + (lane & 31), 2 * ks + (lane >> 5))
                assert direct == 2 * kb * 32 * hd + (base ^ (ks << 5)), (lane, kb, ks)


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_transposed_fragment_xor(hd):
    off = geo(hd)
    dt = hd // 32

    def reads(rb, s, ct, lane):  # byte offsets of the two ds_read_b64_tr_b16
        g, src = lane >> 4, lane & 15
        row = 32 * rb + 16 * s + 4 * (g >> 1) + (src >> 2)
        col = 32 * ct + 16 * (g & 1) + 4 * (src & 3)
        return 2 * (off(row, col >> 3) + (col & 7)), 2 * (off(row + 8, col >> 3) + (col & 7))

    for lane in range(64):
        tb0, tb1 = reads(0, 0, 0, lane)
        for rb in range(2):
            for s in range(2):
                for ct in range(dt):
                    p0, p1 = reads(rb, s, ct, lane)
                    rows = 2 * (32 * rb + 16 * s) * hd
                    assert p0 == rows + (tb0 ^ (64 * ct)), (lane, rb, s, ct)
                    assert p1 == rows + (tb1 ^ (64 * ct)), (lane, rb, s, ct)


def test_identity_catches_a_wrong_swizzle():
    # a swizzle that mixes the 32-row block into the chunk index breaks the
    # row-fragment identity: the check above is not vacuous
    hd, nch = 128, 16

    def off_bad(r, c):
        return r * hd + ((c ^ ((r >> 3) & (nch - 1))) << 3)

    lane, kb, ks = 5, 1, 3
    base = 2 * off_bad(lane & 31, lane >> 5)
    assert 2 * off_bad(kb * 32 + (lane & 31), 2 * ks + (lane >> 5)) != 2 * kb * 32 * hd + (base ^ (ks << 5))
