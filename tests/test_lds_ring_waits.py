"""CPU model of the vector-memory issue order of the LDS-ring GEMM kernels.

The tile kernels copy A (and the e8m0 scales, and in gemm_t32.h B too) into a
ring of LDS slots with ``buffer_load ... lds`` and publish a slot with
``s_waitcnt vmcnt(N)`` + ``s_barrier``: vmcnt(N) returns once at most the N
most recently issued vector-memory operations of the wave are outstanding, so
the copies of the stage being published are complete only if at least N
operations were issued after them.  The counts N are compile-time constants
sized for the steady state of the loop; the prologue and the tile
transitions issue fewer operations between a copy and its wait.  This model
replays each kernel's issue order per wave (register loads of B, ring copies,
epilogue stores) with the kernels' own constants and checks that every wait
that precedes reads of a slot covers that slot's copies.  Inside a k-step
region the compiler may order the region's loads freely, so the model issues
a region's copies last (the fewest followers).

Kernels modelled: gemm_flat.h ``flat_body`` (prologue and main loop; both
its issue orders: B operand loads spread over the k-steps, and the BLDS order
of row-major bf16 B, A copies before the wait and B copies after it),
gemm_t32.h ``gemm_t32_kernel``, gemm_flat_persist.h (prologue, tile
transitions), gemm_skinny_lds.h (S pairs in flight, its up-front, steady and
tail phases, buffer refills; the stream-K form's windows), gemm_lds_persist.h (two stage buffers, the
epilogue's use of a stage buffer, tile transitions), and moe_stage2.h (no
ring: its wave-private epilogue tile).  A wrong count here (the flat
kernel's former prologue wait of (NS - 2) * NDMA) lets the first stage read a
slot whose copies may still be in flight: a timing-dependent wrong tile.
"""
import pytest


class Wave:
    """Issued vector-memory operations of one wave and what the waits so far
    guarantee complete."""

    def __init__(self):
        self.n = 0
        self.done = 0          # operations [0, done) are complete
        self.ops = {}

    def issue(self, tag, k=1):
        for _ in range(k):
            self.ops.setdefault(tag, []).append(self.n)
            self.n += 1

    def wait(self, vmcnt):
        self.done = max(self.done, self.n - vmcnt)

    def complete(self, tag):
        return all(i < self.done for i in self.ops.get(tag, []))


def _parts(ndma):
    """sizes of the three dma_part calls of a stage"""
    dp = (ndma + 2) // 3
    return [max(0, min(ndma, (p + 1) * dp) - p * dp) for p in range(3)]


def flat_prologue_wait(ns, ndma, nb):
    """gemm_flat.h: vmcnt of the prologue wait, (NS - 2 - PRO_WAITED) * NDMA"""
    nbl = 4 * nb
    loads_iter = ndma + nbl
    wait_n = (ns - 3) * loads_iter + ndma + 3 * nb if ns >= 3 else 0
    waited = 0
    for t in range(ns - 2):
        if (ns - 3 - t) * ndma + t * loads_iter + ndma + 3 * nb < wait_n:
            waited = t + 1
    return (ns - 2 - waited) * ndma


def run_flat(ns, ndma, nb, nstages, prologue_wait=flat_prologue_wait):
    """flat_body: B stages 0, 1 into registers, copies of stages 0..NS-2, the
    prologue wait; stage t: three regions (B of stage t+2 k-step r, copies of
    stage t+NS-1 part r), the publishing wait (WAIT_N) for stage t+1, then
    B k-step 3.  Returns the stages whose publishing wait does not cover
    their copies."""
    nbl = 4 * nb
    wait_n = (ns - 3) * (ndma + nbl) + ndma + 3 * nb if ns >= 3 else 0
    w = Wave()
    w.issue(("B", 0), nbl)
    w.issue(("B", 1), nbl)
    for t in range(ns - 1):
        w.issue(("A", t), ndma)
    w.wait(prologue_wait(ns, ndma, nb))
    bad = [] if w.complete(("A", 0)) else [0]
    for t in range(nstages + nstages % 2):
        for r, k in enumerate(_parts(ndma)):
            w.issue(("B", t + 2), nb)
            w.issue(("A", t + ns - 1), k)
        w.wait(wait_n)
        if not w.complete(("A", t + 1)):
            bad.append(t + 1)
        w.issue(("B", t + 2), nb)
    return bad


def flat_blds_waits(ns, ndma):
    """gemm_flat.h with row-major bf16 B copied into two wave-private LDS
    regions (BLDS): per stage the A copies of stage t+NS-1 before the wait,
    the 8 B copies of stage t+2 after it; returns (WAIT_N, prologue vmcnt)
    with the kernel's formulas (PRE_WAIT = NDMA)"""
    loads_iter = ndma + 8
    pre_wait = ndma
    wait_n = ndma
    waited = 0
    for t in range(ns - 2):
        if (ns - 3 - t) * ndma + t * loads_iter + pre_wait < wait_n:
            waited = t + 1
    return wait_n, (ns - 2 - waited) * ndma


def run_flat_blds(ns, ndma, nstages, waits=flat_blds_waits):
    """issue order: prologue B copies of stages 0, 1, A copies of stages
    0..NS-2; stage t: A copies of stage t+NS-1, the wait publishing stage t+1
    (its A and B copies), then the B copies of stage t+2"""
    wait_n, pro = waits(ns, ndma)
    w = Wave()
    w.issue(("B", 0), 8)
    w.issue(("B", 1), 8)
    for t in range(ns - 1):
        w.issue(("A", t), ndma)
    w.wait(pro)
    bad = [] if w.complete(("A", 0)) and w.complete(("B", 0)) else [0]
    for t in range(nstages + nstages % 2):
        w.issue(("A", t + ns - 1), ndma)
        w.wait(wait_n)
        if not (w.complete(("A", t + 1)) and w.complete(("B", t + 1))):
            bad.append(t + 1)
        w.issue(("B", t + 2), 8)
    return bad


def run_t32(ns, ndma, nstages):
    """gemm_t32_kernel: only ring copies (A, B and scales) per stage"""
    wait_n = (ns - 2) * ndma if ns >= 3 else 0
    w = Wave()
    for t in range(ns - 1):
        w.issue(("A", t), ndma)
    w.wait((ns - 2) * ndma)
    bad = [] if w.complete(("A", 0)) else [0]
    for t in range(nstages):
        for k in _parts(ndma):
            w.issue(("A", t + ns - 1), k)
        w.wait(wait_n)
        if not w.complete(("A", t + 1)):
            bad.append(t + 1)
    return bad


def run_persist(ndma, nb, nst, nstages, tiles):
    """gemm_flat_persist.h: 4-slot ring; prologue copies of stages 0, 1, B of
    stages 0, 1, copies of stage 2, NST stand-in stores; per tile nst4 stages
    whose look-ahead moves to the next tile in the last stages (copies from
    stage nst4-3, B from stage nst4-2); epilogue NST stores.  Waits: WAIT_T
    for the first two stages of a tile, WAIT_N after."""
    nbl = 4 * nb
    loads_iter = ndma + nbl
    wait_n = loads_iter + ndma + 3 * nb
    wait_t = min(63, wait_n + nst)
    wait_p = min(63, 2 * ndma + 2 * nbl + nst)
    nst4 = 4 if nstages <= 4 else (8 if nstages <= 8 else (nstages + 3) & ~3)
    w = Wave()
    for t in range(2):
        w.issue(("A", 0, t), ndma)
    w.issue(("B", 0, 0), nbl)
    w.issue(("B", 0, 1), nbl)
    w.issue(("A", 0, 2), ndma)
    w.issue("st", nst)
    w.wait(wait_p)
    bad = [] if w.complete(("A", 0, 0)) else [(0, 0)]
    for it in range(tiles):
        for t in range(nst4):
            dt = (it, t + 3) if t + 3 < nst4 else (it + 1, t + 3 - nst4)
            bt = (it, t + 2) if t + 2 < nst4 else (it + 1, t + 2 - nst4)
            for k in _parts(ndma):
                w.issue(("B",) + bt, nb)
                w.issue(("A",) + dt, k)
            w.wait(wait_t if t < 2 else wait_n)
            pub = (it, t + 1) if t + 1 < nst4 else (it + 1, 0)
            if not w.complete(("A",) + pub):
                bad.append(pub)
            w.issue(("B",) + bt, nb)
        w.issue("st", nst)
        w.wait(63)
    return bad


def _flat_cfg(ka, bm):
    """FlatCfg<KA, BM>: (NS, NDMA) with NB = 2 B tiles per wave"""
    mx = ka != "bf16"
    fa = 2 if ka == "fp8" else 1
    a_ch = bm // 8 * fa
    stage_kb = a_ch + (4 if mx else 0)
    ns = min(4, 160 // stage_kb)
    return ns, a_ch // 4 + (1 if mx else 0)


FLAT_CFGS = [("fp4", 32), ("fp4", 64), ("fp4", 128), ("fp4", 256), ("fp8", 32), ("fp8", 64), ("fp8", 128),
             ("bf16", 128), ("bf16", 256)]


@pytest.mark.parametrize("ka,bm", FLAT_CFGS)
@pytest.mark.parametrize("nstages", [1, 2, 3, 4, 7, 28])
def test_flat_kernel_waits_cover_every_stage(ka, bm, nstages):
    ns, ndma = _flat_cfg(ka, bm)
    assert run_flat(ns, ndma, 2, nstages) == []


@pytest.mark.parametrize("ns", [2, 3, 4])
@pytest.mark.parametrize("ndma", list(range(1, 10)))
def test_flat_kernel_waits_any_ring(ns, ndma):
    assert run_flat(ns, ndma, 2, 12) == []


def test_flat_model_catches_a_short_prologue_wait():
    """The former prologue wait, (NS - 2) * NDMA, covers stage 0 only; with a
    4-slot ring the first stage's wait then does not cover stage 1."""
    def old(ns, ndma, nb):
        return (ns - 2) * ndma

    ns, ndma = _flat_cfg("fp4", 32)
    assert ns == 4
    assert run_flat(ns, ndma, 2, 8, prologue_wait=old) == [1]
    assert run_flat(*_flat_cfg("fp8", 128), 2, 8, prologue_wait=old) == [1]


@pytest.mark.parametrize("ns", [2, 3, 4])
@pytest.mark.parametrize("ndma", list(range(1, 17)))
def test_t32_kernel_waits(ns, ndma):
    assert run_t32(ns, ndma, 10) == []


@pytest.mark.parametrize("ka,bm", [("fp4", 256), ("fp4", 128), ("fp8", 256), ("bf16", 256)])
@pytest.mark.parametrize("eb2", [1, 4, 8])
@pytest.mark.parametrize("nstages", [1, 2, 4, 5, 8, 9, 32])
def test_persistent_kernel_waits(ka, bm, eb2, nstages):
    fa = 2 if ka == "fp8" else 1
    ndma = bm // 8 * fa // 4 + (0 if ka == "bf16" else 1)
    nst = bm * 64 * eb2 // 2048
    assert run_persist(ndma, 2, nst, nstages, tiles=3) == []


def _blds_ring(bm):
    """(NS, NDMA) of the BLDS flat kernel: the A ring gives 64 KiB to the B regions"""
    ns, ndma = _flat_cfg("bf16", bm)
    stage_kb = bm // 8
    ns = ns if ns * stage_kb + 64 <= 160 else (160 - 64) // stage_kb
    return ns, ndma


@pytest.mark.parametrize("bm", [128, 256])
@pytest.mark.parametrize("nstages", [1, 2, 3, 8, 64])
def test_flat_blds_waits(bm, nstages):
    ns, ndma = _blds_ring(bm)
    assert ns == (3 if bm == 256 else 4)
    assert run_flat_blds(ns, ndma, nstages) == []


def test_flat_blds_model_catches_a_loose_wait():
    """A wait that also lets the B copies of the stage being published stay
    outstanding (NDMA + 8) leaves them unchecked."""
    def loose(ns, ndma):
        return ndma + 8, (ns - 2) * ndma

    ns, ndma = _blds_ring(256)
    assert run_flat_blds(ns, ndma, 8, waits=loose) != []


# --------------------------------------------------------------------------
# gemm_skinny_lds.h: S k-pairs in flight per wave, each pair's A copies (and
# row-major B copies or B register loads, and scale loads: LP vector-memory
# operations) in register set / LDS buffer `pair % S`; the wait before a
# pair's MFMAs is vmcnt(after * LP) with `after` = pairs issued after it.
# The model follows the kernel's three phases (all pairs up front when there
# are fewer than S; the steady loop; the tail of R remaining issues) and
# checks that every wait covers its pair, every pair is consumed once and in
# order, and no buffer is refilled before its pair was consumed.

def skinny_lds_lp(ka, mf, nb, bl):
    """vector-memory operations the kernel's issue() emits per k-pair: A
    copies (16*MF rows of ROWB bytes, 64 lanes x 16 B each), B (BL: 2*NB
    whole-line copies of 16*NB rows x 128 B; else two 16-byte halves per
    column block), scale dword loads (one per 32-row group of A and of B)"""
    rowb = 256 if ka == "fp8" else 128
    ncp = 16 * mf * rowb // 1024
    b_ops = (16 * nb * 128 // 1024) if bl else 2 * nb
    scales = 0 if ka == "bf16" else (mf + 1) // 2 + (nb + 1) // 2
    return ncp + b_ops + scales


def run_skinny_lds(s, lp, npairs, w=None, tag=0):
    w = Wave() if w is None else w
    bad = []
    held = {}
    consumed = []

    def issue(pair, buf):
        if buf in held and held[buf] not in consumed:
            bad.append(("refilled before use", pair, buf))
        held[buf] = pair
        w.issue(("P", tag, pair), lp)

    def consume(buf, after):
        pair = held[buf]
        w.wait(after * lp)
        if not w.complete(("P", tag, pair)):
            bad.append(("wait misses", pair))
        consumed.append(pair)

    if npairs < s:
        for u in range(npairs):
            issue(u, u)
        for u in range(npairs):
            consume(u, npairs - 1 - u)
    else:
        for u in range(s - 1):
            issue(u, u)
        t = 0
        while t + 2 * s - 2 < npairs:
            for u in range(s):
                issue(t + u + s - 1, (u + s - 1) % s)
                consume(u, s - 1)
            t += s
        rem = npairs - t - (s - 1)
        assert 0 <= rem < s
        for u in range(s - 1 + rem):
            if u < rem:
                issue(t + u + s - 1, (u + s - 1) % s)
                consume(u % s, s - 1)
            else:
                consume(u % s, s - 2 + rem - u)
    if consumed != list(range(npairs)):
        bad.append(("consumed", consumed))
    return bad


# (KA, MF, NB, S, BL) of every gemm_skinny_alds_kernel instance the registry holds
SKINNY_LDS = [("bf16", 1, 2, 2, True), ("bf16", 2, 2, 2, True), ("bf16", 4, 2, 2, True), ("bf16", 1, 1, 2, True),
              ("bf16", 1, 1, 3, True), ("bf16", 2, 1, 2, True), ("bf16", 2, 2, 2, False), ("bf16", 4, 2, 2, False),
              ("fp4", 2, 2, 2, False), ("fp4", 4, 2, 2, False), ("fp4", 2, 1, 2, False), ("fp8", 2, 2, 2, False)]


@pytest.mark.parametrize("ka,mf,nb,s,bl", SKINNY_LDS)
@pytest.mark.parametrize("npairs", list(range(1, 12)) + [33])
def test_skinny_lds_waits(ka, mf, nb, s, bl, npairs):
    lp = skinny_lds_lp(ka, mf, nb, bl)
    assert (s - 1) * lp < 64          # the kernel's static_assert: vmcnt range
    assert run_skinny_lds(s, lp, npairs) == []


# gemm_skinny_sk_kernel (the stream-K form, row-major bf16 B): each window of
# a workgroup's range runs the same per-wave schedule over the wave's units
# of that window; between windows the wave issues the window's output stores
# (a whole block's stores, or a partial's agent-coherent stores) and waits
# for vmcnt(0), so the next window's waits count its own copies only.
SKINNY_SK = [("bf16", 1, 2, 2, True), ("bf16", 2, 2, 2, True), ("bf16", 4, 2, 2, True)]


@pytest.mark.parametrize("ka,mf,nb,s,bl", SKINNY_SK)
@pytest.mark.parametrize("windows", [[1], [4], [2, 5], [1, 1, 4], [33, 2], [0, 3], [3, 0, 1]])
def test_skinny_sk_waits(ka, mf, nb, s, bl, windows):
    lp = skinny_lds_lp(ka, mf, nb, bl)
    w = Wave()
    for i, npairs in enumerate(windows):
        assert run_skinny_lds(s, lp, npairs, w, tag=i) == []
        w.issue(("store", i), 2)   # the window's output (or partial) stores
        w.wait(0)


def test_skinny_lds_model_catches_a_short_tail_wait():
    """With the tail's last wait one pair short (after - 1), the last pair's
    operations may still be in flight."""
    lp = skinny_lds_lp("fp4", 2, 2, False)

    def short(s, lp, npairs):
        w = Wave()
        for u in range(npairs):
            w.issue(("P", u), lp)
        w.wait(lp)           # should be 0 for the last pair
        return [] if w.complete(("P", npairs - 1)) else ["last pair"]

    assert short(2, lp, 3) == ["last pair"]


# --------------------------------------------------------------------------
# gemm_lds_persist.h and the wave-private buffers: a symmetric trace of one
# wave's LDS events (all waves run the same sequence between barriers).  A
# read of a buffer needs its copies waited for (vmcnt) before a barrier that
# precedes the read; a copy into a buffer needs every earlier read or
# epilogue use of that buffer to be followed by an lgkmcnt(0) wait and a
# barrier before the copy.

def check_trace(events):
    w = Wave()
    bad = []
    copies = {}          # buf -> tags of copies not yet published
    published = set()    # (buf, tag) readable
    pending_use = {}     # buf -> index of the last read / epilogue use not yet fenced
    waited_uses = {}     # buf -> uses completed by an lgkmcnt(0) wait, awaiting a barrier
    for i, ev in enumerate(events):
        kind = ev[0]
        if kind == "dma":
            _, buf, tag, n = ev
            if pending_use.get(buf) is not None or waited_uses.get(buf):
                bad.append(("copy over unfenced use", i, buf))
            w.issue((buf, tag), n)
            copies.setdefault(buf, []).append(tag)
            published.discard((buf, tag))
        elif kind == "wait":
            _, vm, lgkm0 = ev
            w.wait(vm)
            if lgkm0:
                for b, u in list(pending_use.items()):
                    if u is not None:
                        waited_uses[b] = True
                        pending_use[b] = None
        elif kind == "barrier":
            for b, tags in copies.items():
                for t in list(tags):
                    if w.complete((b, t)):
                        published.add((b, t))
                        tags.remove(t)
            waited_uses.clear()
        elif kind in ("read", "ep"):
            _, buf, tag = ev
            if kind == "read" and (buf, tag) not in published:
                bad.append(("read before publish", i, buf, tag))
            pending_use[buf] = i
    return bad


def lds_persist_trace(nst, tiles, ndma=16):
    """gemm_lds_persist_kernel: two stage buffers; stage t (buffer t % 2)
    issues the copies of stage t+1 into the other buffer, reads its own
    buffer over 4 k-steps, waits vmcnt(0) lgkmcnt(0) + barrier, reads k-step 0
    of the next stage; the last stage of a tile copies the next tile's stage
    0; the epilogue stages the output through buffer 1, then lgkmcnt(0) +
    barrier.  nst is even (the kernel pads K to an even stage count)."""
    ev = [("dma", 0, (0, 0), ndma), ("wait", 0, True), ("barrier",), ("read", 0, (0, 0))]
    for it in range(tiles):
        for t in range(nst):
            buf = t % 2
            nxt = (it, t + 1) if t + 1 < nst else (it + 1, 0)
            ev.append(("dma", buf ^ 1, nxt, ndma))
            ev += [("read", buf, (it, t))] * 3
            ev += [("wait", 0, True), ("barrier",), ("read", buf ^ 1, nxt)]
        ev += [("ep", 1, None), ("wait", 63, True), ("barrier",)]
    return ev


@pytest.mark.parametrize("nst", [2, 4, 8, 64])
@pytest.mark.parametrize("tiles", [1, 2, 5])
def test_lds_persist_buffers(nst, tiles):
    assert check_trace(lds_persist_trace(nst, tiles)) == []


def test_lds_persist_model_catches_an_early_copy():
    """Issuing the next stage's copies before the barrier that ends the reads
    of that buffer (here: an odd stage count, so the tile's first copy lands in
    the buffer the epilogue just used, before its barrier) is flagged."""
    ev = lds_persist_trace(2, 2)
    i = ev.index(("ep", 1, None))
    bad_ev = ev[:i + 1] + [("dma", 1, ("x", 0), 16)] + ev[i + 1:]
    assert check_trace(bad_ev) != []


def test_moe_stage2_needs_no_ring_waits():
    """moe_stage2.h keeps A and B in registers (the compiler orders their
    loads and uses) and uses LDS only for a wave-private epilogue tile that the
    same wave writes and then reads back: LDS operations of one wave complete
    in issue order, so no wait or barrier publishes anything.  The model of
    that tile: every read follows the wave's own write of the same bytes.
    The granule swizzle uses row bits 1-3, so each 8-byte store instruction
    (32 rows of 16 bytes) puts at most two rows on one 16-byte granule of the
    256-byte bank line (the floor for 512 bytes)."""
    bm = 32

    def swz(r):
        return (r >> 1) & 7

    written = set()
    for i in range(bm // 32):
        for j in range(2):
            for q in range(4):
                hits = {}
                for lane in range(64):
                    r = 32 * i + (lane & 31)
                    cc = 8 * j + 2 * q + (lane >> 5)
                    off = ((cc >> 1) ^ swz(r)) * 16 + (cc & 1) * 8
                    written.add((r, off))
                    written.add((r, off + 4))
                    g = ((r * 128 + off) % 256) // 16
                    hits.setdefault(g, set()).add(r)
                assert max(len(v) for v in hits.values()) <= 2
    for r0 in range(0, bm, 8):
        for lane in range(64):
            r = r0 + (lane >> 3)
            base = ((lane & 7) ^ swz(r)) * 16
            for b in range(0, 16, 4):
                assert (r, base + b) in written
