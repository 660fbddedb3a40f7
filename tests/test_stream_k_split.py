"""CPU model of the stream-K skinny kernel's work split
(gemm_skinny_sk_kernel in aiter_amd/csrc/gemm_skinny_lds.h): the index
arithmetic of the kernel, restated for every workgroup of a grid, must
cover each (column block, k-pair) unit exactly once, give every partial
segment its own workspace slot, let the reader find exactly the slots the
writers filled (in range order), and count per block as many arrivals as
the reader expects, so that the last arrival is the one that sums."""
import itertools


def _ranges(U, G):
    return [(g * U // G, (g + 1) * U // G) for g in range(G)]


def _owner(x, U, G):
    return ((x + 1) * G - 1) // U


def _walk(nblk, T, G, NW=8):
    """What each workgroup of the kernel does: (g, block, lo, hi, whole,
    slot) per segment, and the units each wave takes."""
    U = nblk * T
    segs, units = [], []
    for g, (lo0, hi) in enumerate(_ranges(U, G)):
        x = lo0
        while x < hi:
            b0 = x // T
            xe = min(hi, (b0 + 2) * T)
            xb = min(xe, (b0 + 1) * T)
            for w in range(NW):
                ub = x + w
                npairs = (xe - ub + NW - 1) // NW if ub < xe else 0
                tsw = (xb - ub + NW - 1) // NW if xb > ub else 0
                for t in range(npairs):
                    u = ub + t * NW
                    blk = b0 if u < xb else b0 + 1
                    # the register set the unit lands in matches its block
                    assert (t >= tsw) == (blk == b0 + 1)
                    units.append((blk, u - blk * T))
            for st in (0, 1):
                slo, shi = (xb, xe) if st else (x, xb)
                if slo >= shi:
                    continue
                blk = b0 + st
                whole = slo == blk * T and shi == (blk + 1) * T
                which = 0 if slo == lo0 else 1
                segs.append((g, blk, slo, shi, whole, (g, which)))
            x = xe
    return U, segs, units


def test_every_unit_once_and_slots_consistent():
    for nblk, T, G in itertools.chain(
            [(224, 32, 256), (1, 2, 256), (2, 4, 256), (896, 8, 256), (448, 64, 256), (65, 16, 256),
             (128, 112, 256), (3, 1, 5), (7, 3, 4), (8, 112, 64), (66, 112, 256), (1, 32, 8)],
            ((n, t, g) for n in (1, 2, 3, 5, 17) for t in (1, 2, 3, 16) for g in (1, 2, 7, 64))):
        G = min(G, nblk * T)
        U, segs, units = _walk(nblk, T, G)
        assert sorted(units) == [(b, p) for b in range(nblk) for p in range(T)], (nblk, T, G)
        slots = [s[5] for s in segs if not s[4]]
        assert len(slots) == len(set(slots)), (nblk, T, G)
        for blk in range(nblk):
            parts = [s for s in segs if s[1] == blk]
            x0 = blk * T
            if len(parts) == 1 and parts[0][4]:
                continue
            assert all(not s[4] for s in parts)
            gf, gl = _owner(x0, U, G), _owner(x0 + T - 1, U, G)
            # the reader's slots, in range order, are the writers' slots in k order
            read = [(gg, 1 if gg * U // G < x0 else 0) for gg in range(gf, gl + 1)]
            written = [s[5] for s in sorted(parts, key=lambda s: s[2])]
            assert read == written, (nblk, T, G, blk)
            # contiguous cover of the block by the segments
            spans = sorted((s[2], s[3]) for s in parts)
            assert spans[0][0] == x0 and spans[-1][1] == x0 + T
            assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))


def test_decode_shape_balance():
    """N = 7168, K = 2048 at 32 columns per block: 224 blocks x 32 k-pairs on
    256 workgroups, 28 units each (against 32 per block-sized workgroup)."""
    U, segs, _ = _walk(224, 32, 256)
    per = [sum(s[3] - s[2] for s in segs if s[0] == g) for g in range(256)]
    assert min(per) == max(per) == 28
    assert max(sum(1 for s in segs if s[1] == b) for b in range(224)) == 2
