"""CPU replay of the address arithmetic of the HIP kernels (test infrastructure, no GPU).

Each ``replay_*`` function restates, for one C-ABI entry point, what the host side launches (the
variant, grid and block schedule the dispatch code picks for the given shapes) and every global
load, store and global->LDS DMA those kernels issue, plus their LDS reads and writes, as byte
offsets.  The offsets are computed with numpy over all threads of a block; over the blocks, the
schedule decode is evaluated for every block (each (band, row tile, sub-tile) unit must be hit
exactly once) and the memory accesses for every band and sub-tile at the first and last row tile.
K loops move a per-lane offset by a fixed stride per step, so their extremes are the first two
steps and the last one, which are the steps evaluated.

``Bounds.violations()`` lists every buffer whose touched byte range leaves the buffer the caller
allocates for the entry point (sizes from the C-ABI contract in include/pymsst_amd.h).  Every
formula below cites the kernel source it restates (pymsst_amd/csrc/<file>:<kernel>).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

WAVE = 64
XCDS = 8
CHUNK_K = 32
GEMM_THREADS = 256
LDS_PITCH16 = CHUNK_K + 8  # 16-bit LDS row pitch of gemm.h (elements)
LDS_PITCH32 = CHUNK_K + 1


# ----------------------------------------------------------------------------- recorder


@dataclass
class Bounds:
    sizes: dict
    lo: dict = field(default_factory=dict)
    hi: dict = field(default_factory=dict)
    notes: list = field(default_factory=list)

    def touch(self, buf: str, off, width: int, mask=None) -> None:
        """Accesses of ``width`` bytes at byte offsets ``off`` (where ``mask``) of buffer ``buf``."""
        off = np.asarray(off, dtype=np.int64)
        if mask is not None:
            off = off[np.broadcast_to(np.asarray(mask, dtype=bool), off.shape)]
        if off.size == 0:
            return
        lo, hi = int(off.min()), int(off.max()) + int(width)
        self.lo[buf] = min(self.lo.get(buf, lo), lo)
        self.hi[buf] = max(self.hi.get(buf, hi), hi)

    def fail(self, msg: str) -> None:
        self.notes.append(msg)

    def violations(self) -> list[str]:
        out = list(self.notes)
        for buf in self.lo:
            size = self.sizes[buf]
            if self.lo[buf] < 0 or self.hi[buf] > size:
                out.append(f"{buf}: bytes [{self.lo[buf]}, {self.hi[buf]}) outside [0, {size})")
        return out


def steps(nk: int) -> list[int]:
    """K-loop steps whose offsets bound every step's: 0, 1 and the last."""
    return sorted({c for c in (0, 1, nk - 1) if 0 <= c < nk})


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


# ----------------------------------------------------------------------------- device helpers


def swz_k(r):  # dma_gemm.h
    return ((r >> 1) ^ (r >> 3)) & 3


def swz_mn(k):  # dma_gemm.h
    return 2 * (k & 3)


def swz_mn_p(pitch: int, k):  # dma_gemm.h swz_mn_p<PITCH>
    if pitch == 512:
        return 2 * ((k & 3) | (((k >> 3) & 3) << 2))
    return swz_mn(k)


def frag_mn_addr(region, c0, pitch, lane, p512=False):  # dma_gemm.h frag_mn_addr / frag_mn_addr_p
    j, g = lane & 15, lane >> 4
    k = 8 * g + (j >> 2)
    col = c0 + 4 * (j & 3)
    unit = col >> 3
    sw = swz_mn_p(pitch, k) if p512 else swz_mn(k)
    return region + k * pitch + 16 * (unit ^ sw) + 2 * (col & 7)


def frag_k_addr(region, r0, lane):  # dma_gemm.h
    rr, g = lane & 15, lane >> 4
    return region + (r0 + rr) * 64 + 16 * (g ^ swz_k(rr))


def lds_index16(r, k):  # gemm.h lds_index for 16-bit types (elements)
    return r * LDS_PITCH16 + ((((k >> 3) ^ ((r >> 4) & 3)) << 3) | (k & 7))


def xcd_decode(groups: int, members: int):
    """gemm.h XcdGrid: blocks() and xcd_block(); returns (group, member, valid) per block."""
    nblocks = cdiv(groups, XCDS) * XCDS * members
    b = np.arange(nblocks, dtype=np.int64)
    r = b // XCDS
    member = r % members
    group = (r // members) * XCDS + b % XCDS
    return group, member, group < groups


@dataclass
class BandSched:
    gs: list
    cumb: list
    bstart: list
    m_tiles: int
    per_xcd: int


def build_band_sched(nb: int, m_tiles: int, units, cost=lambda b: 1):
    """dma_gemm.h build_band_sched (returns None where the host falls back)."""
    if nb > 256 or m_tiles <= 0:
        return None
    cumb = [0]
    total = total_cost = ucmax = 0
    for b in range(nb):
        u = int(units(b))
        uc = u * int(cost(b))
        ucmax = max(ucmax, uc)
        total += u * m_tiles
        total_cost += uc * m_tiles
        if total >= 1 << 31:
            return None
        cumb.append(total)

    def ranges(cap, fill, gs, bstart):
        x = 0
        acc = g = 0
        if fill:
            gs[0] = 0
            bstart[0] = 0
        for b in range(nb):
            ch = (cumb[b + 1] - cumb[b]) // m_tiles
            uc = ch * int(cost(b))
            for _ in range(m_tiles):
                if acc + uc > cap:
                    x += 1
                    acc = 0
                    if fill and x < XCDS:
                        gs[x] = g
                        bstart[x] = b
                acc += uc
                g += ch
        if fill:
            for y in range(x + 1, XCDS + 1):
                gs[y] = total
                if y < XCDS:
                    bstart[y] = nb - 1
        return x + 1

    lo, hi = ucmax, max(total_cost, ucmax)
    while lo < hi:
        mid = (lo + hi) // 2
        if ranges(mid, False, None, None) <= XCDS:
            hi = mid
        else:
            lo = mid + 1
    gs = [0] * (XCDS + 1)
    bstart = [0] * XCDS
    ranges(lo, True, gs, bstart)
    per_xcd = max(gs[y + 1] - gs[y] for y in range(XCDS))
    return BandSched(gs, cumb, bstart, m_tiles, per_xcd)


def build_even_sched(nb: int, m_tiles: int, units):
    """dma_gemm.h build_even_sched: canonical blocks split evenly over the XCDs."""
    if nb > 256 or m_tiles <= 0:
        return None
    cumb = [0]
    for b in range(nb):
        cumb.append(cumb[-1] + int(units(b)) * m_tiles)
    total = cumb[-1]
    gs = [total * x // XCDS for x in range(XCDS + 1)]
    bstart = []
    b = 0
    for x in range(XCDS):
        while b < nb - 1 and cumb[b + 1] <= gs[x]:
            b += 1
        bstart.append(b)
    per_xcd = max(gs[x + 1] - gs[x] for x in range(XCDS))
    return BandSched(gs, cumb, bstart, m_tiles, per_xcd)


def sched_decode(sc: BandSched, nb: int, units, last_first: bool, bnd: Bounds, what: str):
    """dma_gemm.h sched_block over every block of the grid; checks that the units are covered once
    and that the forward band search starting at bstart finds each block's band."""
    nblocks = sc.per_xcd * XCDS
    seen = np.zeros(sc.cumb[-1], dtype=np.int64)
    out = []
    for blk in range(nblocks):
        xcd, local = blk % XCDS, blk // XCDS
        if sc.gs[xcd] + local >= sc.gs[xcd + 1]:
            continue
        gb = sc.gs[xcd + 1] - 1 - local if last_first else sc.gs[xcd] + local
        b = sc.bstart[xcd]
        if b >= nb or sc.cumb[b] > gb:
            bnd.fail(f"{what}: block {blk} starts its band search past its band")
            continue
        while gb >= sc.cumb[b + 1]:
            b += 1
            if b >= nb:
                break
        if b >= nb:
            bnd.fail(f"{what}: block {blk} decodes past the last band")
            continue
        per_unit = (sc.cumb[b + 1] - sc.cumb[b]) // sc.m_tiles
        within = gb - sc.cumb[b]
        mt, sub = within // per_unit, within % per_unit
        if per_unit != units(b) or not (0 <= mt < sc.m_tiles):
            bnd.fail(f"{what}: block {blk} decodes to band {b} row tile {mt} unit size {per_unit}")
        seen[gb] += 1
        out.append((b, mt, sub))
    if seen.size and (seen.min() != 1 or seen.max() != 1):
        bnd.fail(f"{what}: {int((seen != 1).sum())} schedule units not covered exactly once")
    return out


# ----------------------------------------------------------------------------- gemm.h loaders


def krow_rows(tid, rows):
    """Tile rows of each thread's quads in a KRowLoader of ``rows`` rows: [threads, quads]."""
    kq = rows * (CHUNK_K // 4) // GEMM_THREADS
    return (tid[:, None] + np.arange(kq)[None, :] * GEMM_THREADS) // (CHUNK_K // 4)


def krow_loader(bnd, buf, esz, base_el, stride, rows_valid, k_valid, rows, v4, kbeg, nk, tid, row_map=None):
    """gemm.h KRowLoader: thread t moves quads (r, k) = ((t + 256 i) / 8, 4 (t % 8)) of every chunk;
    rows past rows_valid are clamped (interior) or masked (edge chunk).  ``row_map`` = (src, row_ok)
    arrays replace the default map (a loader's own prepare())."""
    r = krow_rows(tid, rows)
    lane_k = (tid % (CHUNK_K // 4)) * 4
    if row_map is None:
        src = np.minimum(r, rows_valid - 1)
        row_ok = r < rows_valid
    else:
        src, row_ok = row_map
    for c in steps(nk):
        k = kbeg + CHUNK_K * c + lane_k[:, None]
        edge = (c == 0 and kbeg < 0) or not v4
        if not edge:
            bnd.touch(buf, (base_el + src * stride + k) * esz, 4 * esz)
        elif v4:
            ok = row_ok & (k >= 0) & (k < k_valid)
            bnd.touch(buf, np.where(ok, base_el + src * stride + k, base_el) * esz, 4 * esz)
        else:
            for j in range(4):
                ok = row_ok & (k + j >= 0) & (k + j < k_valid)
                bnd.touch(buf, np.where(ok, base_el + src * stride + k + j, base_el) * esz, esz)


def mn_loader(bnd, buf, esz, base_el, kstride, mn_valid, k_valid, rows, v4, kbeg, nk, tid):
    """gemm.h MNLoader: element (k, mn) = base[k * kstride + mn]; thread t owns mn quad 4 (t % (ROWS/4))
    and k rows (t / (ROWS/4)) * KB .. + KB - 1 of each chunk (KB = ROWS / 32)."""
    qpk = rows // 4
    kb_n = rows // 32
    mn = (tid % qpk) * 4
    kb = (tid // qpk) * kb_n
    mn_src = np.where(v4 & (mn >= mn_valid), mn_valid - 4, mn)
    for c in steps(nk):
        for t in range(kb_n):
            k = kbeg + CHUNK_K * c + kb + t
            edge = (c == 0 and kbeg < 0) or not v4
            if not edge:
                bnd.touch(buf, (base_el + k * kstride + mn_src) * esz, 4 * esz)
            elif v4:
                kok = (k >= 0) & (k < k_valid)
                bnd.touch(buf, np.where(kok, base_el + k * kstride + mn_src, base_el) * esz, 4 * esz)
            else:
                kok = (k >= 0) & (k < k_valid)
                kc = np.where(kok, k, 0)
                for j in range(4):
                    ok = kok & (mn + j < mn_valid)
                    bnd.touch(buf, np.where(ok, base_el + kc * kstride + mn + j, base_el) * esz, esz)


def gemm_lds_bytes(esz, br, bc):
    return 2 * (br + bc) * (LDS_PITCH16 if esz == 2 else LDS_PITCH32) * esz


# ----------------------------------------------------------------------------- band split


def _offs(widths):
    return np.concatenate([[0], np.cumsum(widths)]).astype(np.int64)


def tile_capacity(o):
    return min(4, cdiv(o, 64))


def replay_band_split_forward(widths, M, O, esz, *, norm=True, x_stride=None, has_bias=True, act_tanh=False):
    """band_split.hip launch_fwd + bs_fwd_kernel (also the grouped linear forward when norm=False)."""
    nb, F = len(widths), int(sum(widths))
    x_stride = F if x_stride is None else x_stride
    offs = _offs(widths)
    sizes = {"x": ((M - 1) * x_stride + F) * esz, "gamma": F * esz, "weight": O * F * esz,
             "bias": nb * O * esz, "out": M * nb * O * esz, "inv_norm": M * nb * 4, "offsets": (nb + 1) * 8,
             "lds": 0}
    bnd = Bounds(sizes)
    vec4 = all(w % 4 == 0 for w in widths) and x_stride % 4 == 0
    ovec4 = O % 4 == 0
    ovec8 = esz == 2 and ovec4 and O % 8 == 0
    TO = tile_capacity(O) if vec4 else 4
    OT = 64 * TO
    cap = 64 * tile_capacity(O)
    sizes["lds"] = gemm_lds_bytes(esz, OT, 64) + 64 * 4
    mtiles, oz = cdiv(M, 64), cdiv(O, cap)
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    for by in range(nb):
        band = nb - 1 - by
        bnd.touch("offsets", np.array([band, band + 1]) * 8, 8)
        off, I = int(offs[band]), int(widths[band])
        nk = cdiv(I, CHUNK_K)
        kbeg = I - nk * CHUNK_K
        for bx in sorted({0, mtiles - 1}):
            m0 = bx * 64
            rv = min(M - m0, 64)
            for bz in range(oz):
                oc = bz * OT
                # A: weight rows oc .. of band b ([O, I_b] at O * off), K = I
                krow_loader(bnd, "weight", esz, O * off + oc * I, I, O - oc, I, OT, vec4, kbeg, nk, tid)
                # B: x rows (clamped) of the band; gamma of the thread's k quad
                krow_loader(bnd, "x", esz, m0 * x_stride + off, x_stride, rv, I, 64, vec4, kbeg, nk, tid)
                if norm:
                    for c in steps(nk):
                        k = kbeg + CHUNK_K * c + (tid % 8) * 4
                        if (c == 0 and kbeg < 0) or not vec4:
                            for j in range(4):
                                ok = (k + j >= 0) & (k + j < I)
                                bnd.touch("gamma", np.where(ok, off + k + j, off) * esz, esz)
                        else:
                            bnd.touch("gamma", (off + k) * esz, 4 * esz)
                    r = np.arange(64)
                    if bz == 0:
                        bnd.touch("inv_norm", ((m0 + r) * nb + band) * 4, 4, r < rv)
                # epilogue
                for t in range(TO):
                    o = oc + wave * 16 * TO + t * 16 + 4 * (lane >> 4)
                    ok = o < O
                    if has_bias:
                        if ovec4:
                            bnd.touch("bias", (band * O + o) * esz, 4 * esz, ok)
                        else:
                            for rr in range(4):
                                bnd.touch("bias", (band * O + o + rr) * esz, esz, ok & (o + rr < O))
                    if ovec8:
                        kop = OT + 8
                        ol = wave * 16 * TO + t * 16 + 4 * (lane >> 4)
                        for j in range(4):
                            m = j * 16 + (lane & 15)
                            bnd.touch("lds", (m * kop + ol) * esz, 4 * esz, ok)
                    else:
                        for j in range(4):
                            m = j * 16 + (lane & 15)
                            okm = ok & (m < rv)
                            if ovec4:
                                bnd.touch("out", (((m0 + m) * nb + band) * O + o) * esz, 4 * esz, okm)
                            else:
                                for rr in range(4):
                                    bnd.touch("out", (((m0 + m) * nb + band) * O + o + rr) * esz, esz,
                                              okm & (o + rr < O))
                if ovec8:
                    kop = OT + 8
                    ov = min(O - oc, OT)
                    q = np.arange(64 * (ov // 8))
                    m, cc = q // (ov // 8), (q % (ov // 8)) * 8
                    okm = m < rv
                    bnd.touch("lds", (m * kop + cc) * esz, 16, okm)
                    bnd.touch("out", (((m0 + m) * nb + band) * O + oc + cc) * esz, 16, okm)
    return bnd


def replay_band_split_backward(widths, M, O, esz, *, has_bias=True, grouped=False, even_dx=False):
    """band_split.hip launch_bwd (saved input: the split dx kernel writing t = gs * gamma and the dot
    partials, bs_dx_finish_kernel, the DMA-ring or register dW kernel, col_sum) or launch_grouped_bwd
    (grouped=True: the norm-free dx and dW kernels)."""
    nb, F = len(widths), int(sum(widths))
    offs = _offs(widths)
    m_tiles = cdiv(M, 64)
    dgp = cdiv(m_tiles * F * 4, 256) * 256
    pitch = F // 64 + nb + 1
    pdb = cdiv(M * pitch * 4, 256) * 256
    tbb = cdiv(M * F * 4, 256) * 256
    sizes = {"dy": M * nb * O * esz, "x": M * F * esz, "inv_norm": M * nb * 4, "gamma": F * esz,
             "weight": O * F * esz, "dx": M * F * esz, "dgamma": F * esz, "dw": O * F * esz,
             "db": nb * O * esz, "offsets": (nb + 1) * 8,
             "workspace": 0 if grouped else dgp + pdb + tbb, "lds": 0, "lds_finish": 2 * 64 * 4}
    bnd = Bounds(sizes)
    vec4 = all(w % 4 == 0 for w in widths)
    ovec4 = O % 4 == 0
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    norm = not grouped
    # -- dx of the grouped linear on grouped_dx.hip (16-bit, uniform supported widths)
    if grouped and esz == 2 and M > 0 and len(set(widths)) == 1 and widths[0] in GDX_TILES and O % 32 == 0 \
            and O >= 64:
        _replay_glin_dx(bnd, nb, widths[0], O, M)
        M_dx = 0  # the register-path dx kernel below does not run
    else:
        M_dx = M
    # -- dx (one block per (band, 64-wide input chunk, 64 rows))
    max_ich = cdiv(max(widths), 64)
    sizes["lds"] = gemm_lds_bytes(esz, 64, 64) + 64 * 4 + 4 * 64 * 4
    if M_dx > 0:
        # norm: the even schedule over the existing (band, row tile, chunk) blocks (the XcdGrid of
        # NB * max_ichunks groups past 256 bands); grouped: the XcdGrid (all groups one width)
        sc = build_even_sched(nb, m_tiles, lambda b: cdiv(widths[b], 64)) if norm or even_dx else None
        if sc is not None:
            sched_decode(sc, nb, lambda b: cdiv(widths[b], 64), True, bnd, "bs_bwd_dx")
        else:
            grp, mt, valid = xcd_decode(nb * max_ich, m_tiles)
            if np.any(mt[valid] >= m_tiles):
                bnd.fail("dx: member out of range")
        v4 = vec4 and ovec4
        for band in range(nb):
            off, I = int(offs[band]), int(widths[band])
            for ich in range(max_ich):
                i0 = ich * 64
                if i0 >= I:
                    continue
                for mtile in sorted({0, m_tiles - 1}):
                    m0 = mtile * 64
                    rv = min(M - m0, 64)
                    r64 = np.arange(64)
                    if norm:
                        bnd.touch("inv_norm", ((m0 + r64) * nb + band) * 4, 4, r64 < rv)
                        # dot partial of the chunk: row m, column off / 64 + band + chunk
                        bnd.touch("workspace", dgp + ((m0 + r64) * pitch + off // 64 + band + ich) * 4, 4, r64 < rv)
                    nk = cdiv(O, CHUNK_K)
                    kbeg = O - nk * CHUNK_K
                    mn_loader(bnd, "weight", esz, O * off + i0, I, I - i0, O, 64, v4, kbeg, nk, tid)
                    krow_loader(bnd, "dy", esz, (m0 * nb + band) * O, nb * O, rv, O, 64, v4, kbeg, nk, tid)
                    il = i0 + wave * 16 + 4 * (lane >> 4)
                    for j in range(4):
                        m = j * 16 + (lane & 15)
                        ok = (m < rv) & (il < I)
                        if norm:
                            for r in range(4):
                                gi = np.where(il + r < I, off + il + r, off)
                                bnd.touch("gamma", gi * esz, esz, il + r < I)
                        e = (m0 + m) * F + off + il
                        if vec4:
                            if norm:
                                bnd.touch("x", e * esz, 4 * esz, ok)
                                bnd.touch("workspace", dgp + pdb + e * 4, 16, ok)
                            else:
                                bnd.touch("dx", e * esz, 4 * esz, ok)
                        else:
                            for r in range(4):
                                okr = ok & (il + r < I)
                                if norm:
                                    bnd.touch("x", (e + r) * esz, esz, okr)
                                    bnd.touch("workspace", dgp + pdb + (e + r) * 4, 4, okr)
                                else:
                                    bnd.touch("dx", (e + r) * esz, esz, okr)
                    if norm:
                        for r in range(4):
                            bnd.touch("workspace", (mtile * F + off + il + r) * 4, 4,
                                      ((lane & 15) == 0) & (il + r < I))
        # -- finish: the dx kernel's blocks (band, 64-wide chunk, 64 rows); with the DMA dW kernel and the
        # dx schedule they are that kernel's tail blocks, decoded at blockIdx.x minus its scheduled
        # blocks (a multiple of 8): the same decode and addresses
        if norm:
            for band in range(nb):
                off, I = int(offs[band]), int(widths[band])
                nch = cdiv(I, 64)
                for ich in range(max_ich):
                    i0 = ich * 64
                    if i0 >= I:
                        continue
                    for mtile in sorted({0, m_tiles - 1}):
                        m0 = mtile * 64
                        rv = min(M - m0, 64)
                        r, part = tid >> 2, tid & 3
                        for c0 in range(4):
                            for c in range(c0, nch, 4):
                                ok = (r < rv) & (part == c0)
                                bnd.touch("workspace", dgp + ((m0 + r) * pitch + off // 64 + band + c) * 4, 4, ok)
                        okw = (part == 0) & (r < rv)
                        bnd.touch("inv_norm", ((m0 + r) * nb + band) * 4, 4, okw)
                        bnd.touch("lds_finish", r * 4, 4, okw)
                        bnd.touch("lds_finish", 64 * 4 + r * 4, 4, okw)
                        k = i0 + 4 * (tid & 15)
                        live = k < I
                        for j in range(4):
                            rr = (tid >> 4) + 16 * j
                            rc = np.where(rr < rv, rr, rv - 1)
                            okr = live & (rr < rv)
                            bnd.touch("lds_finish", np.minimum(rr, 63) * 4, 4, okr)
                            bnd.touch("lds_finish", 64 * 4 + np.minimum(rr, 63) * 4, 4, okr)
                            if vec4:
                                e = (m0 + rc) * F + off + k
                                bnd.touch("workspace", dgp + pdb + e * 4, 16, live)
                                bnd.touch("x", e * esz, 4 * esz, live)
                                bnd.touch("dx", ((m0 + rr) * F + off + k) * esz, 4 * esz, okr)
                            else:
                                e = (m0 + rr) * F + off + k
                                for q in range(4):
                                    okq = okr & (k + q < I)
                                    bnd.touch("workspace", dgp + pdb + (e + q) * 4, 4, okq)
                                    bnd.touch("x", (e + q) * esz, esz, okq)
                                    bnd.touch("dx", (e + q) * esz, esz, okq)
    # -- dW
    dma = (not grouped) and esz == 2 and M >= 64 and vec4 and O % 8 == 0
    uniform_dw = grouped and esz == 2 and M >= CHUNK_K and len(set(widths)) == 1 and widths[0] % 64 == 0 \
        and O % 8 == 0
    if dma:
        _replay_bs_dw_dma(bnd, widths, offs, M, O, esz, has_bias)
    elif uniform_dw:  # the mask-estimator DMA dW kernel with HT = 64 on bands of width 2 I_b = O
        _replay_me_dw_dma(bnd, [O // 2] * nb, _offs([O // 2] * nb), M, widths[0], esz, 64, "dy", "x", "dw",
                          "db" if has_bias else None, "lds_dw", JT=dw_jt(nb, widths[0], O))
    else:
        _replay_bs_dw_reg(bnd, widths, offs, M, O, esz, has_bias, norm, vec4 and ovec4)
    if norm:
        # col_sum_kernel over the m_tiles x F partials -> dgamma
        _replay_col_sum(bnd, "workspace", m_tiles, F, "dgamma", esz)
    return bnd


ROWSUM_MAX_F = 16384  # band_split.hip kRowSumMaxF


def _replay_band_rowsum_row(bnd, widths, offs, M, x_stride, mode, gbuf):
    """band_split.hip band_rowsum_row_kernel: one block per row; thread t's quads t + 256 k (x, and g,
    gamma for MODE 1), the quad sums and piece sums in LDS (piece p of band b at off_b / 64 + b + c),
    out[m, b].  Rows 0 and M - 1 bound every block's offsets."""
    nb, F = len(widths), int(sum(widths))
    nq = F // 4
    npieces = F // 64 + nb + 1
    bnd.sizes.setdefault("lds_qsum", ROWSUM_MAX_F)
    bnd.sizes.setdefault("lds_psum", (ROWSUM_MAX_F // 64 + 256 + 1) * 4)
    q = np.arange(nq)
    p = np.arange(npieces)
    key = offs[:-1] // 64 + np.arange(nb)
    band = np.searchsorted(key, p, side="right") - 1
    if np.any(band < 0) or np.any(band >= nb):
        bnd.fail("rowsum_row: piece band lookup out of range")
    band = np.clip(band, 0, nb - 1)
    q0 = offs[band] // 4 + 16 * (p - key[band])
    q1 = np.minimum(q0 + 16, offs[band + 1] // 4)
    if np.any(q0[q1 > q0] < 0) or np.any(q1 > nq):
        bnd.fail("rowsum_row: a piece reads quads outside the row")
    covered = np.zeros(nq, dtype=np.int64)
    for a_, b_ in zip(q0, q1):
        covered[a_:b_] += 1
    if np.any(covered != 1):
        bnd.fail("rowsum_row: the pieces do not cover every quad exactly once")
    bnd.touch("lds_psum", p * 4, 4)
    bnd.touch("lds_qsum", q * 4, 4)
    for m in sorted({0, M - 1}):
        bnd.touch("x", (m * x_stride + 4 * q) * 4, 16)
        if mode == 1:
            bnd.touch(gbuf, (m * F + 4 * q) * 2, 8)
            bnd.touch("gamma", 4 * q * 4, 16)
        bnd.touch("inv_norm" if mode == 0 else "dot", (m * nb + np.arange(nb)) * 4, 4)


def _replay_band_rowsum(bnd, widths, offs, M, x_stride, mode, gbuf):
    """band_split.hip launch_rowsum: band_rowsum_row_kernel where it fits, else band_rowsum_kernel: one
    wave per (64-row tile, band), lane = row (clamped to the last row); MODE 0 reads x, MODE 1 also g
    (16-bit, pitch F) and gamma; writes out[m, b] for m < M."""
    nb, F = len(widths), int(sum(widths))
    v4 = all(w % 4 == 0 for w in widths) and x_stride % 4 == 0
    if v4 and F <= ROWSUM_MAX_F and nb <= 256:
        _replay_band_rowsum_row(bnd, widths, offs, M, x_stride, mode, gbuf)
        return
    m_tiles = cdiv(M, 64)
    waves = m_tiles * nb
    wid = np.arange(cdiv(waves, 4) * 4)
    band = nb - 1 - wid // m_tiles
    live_w = band >= 0
    if np.any(wid[live_w] // m_tiles >= nb):
        bnd.fail("rowsum: band out of range")
    lane = np.arange(64)
    for w in [(nb - 1 - b) * m_tiles + mt for b in range(nb) for mt in sorted({0, m_tiles - 1})]:
        b = nb - 1 - int(w) // m_tiles
        mt = int(w) % m_tiles
        m = mt * 64 + lane
        mr = np.minimum(m, M - 1)
        off, I = int(offs[b]), int(widths[b])
        bnd.touch("offsets", np.array([b, b + 1]) * 8, 8)
        step = 4 if v4 else 1
        for i in sorted({0, I - step}):
            bnd.touch("x", (mr * x_stride + off + i) * 4, 4 * step)
            if mode == 1:
                bnd.touch(gbuf, (mr * F + off + i) * 2, 2 * step)
                bnd.touch("gamma", (off + i) * 4, 4 * step)
        bnd.touch("inv_norm" if mode == 0 else "dot", (m * nb + b) * 4, 4, m < M)
    # every (band, row tile) is one wave's: the decode is a bijection
    seen = {(nb - 1 - int(w) // m_tiles, int(w) % m_tiles) for w in wid[live_w]}
    if len(seen) != waves:
        bnd.fail("rowsum: a (band, row tile) is missed or run twice")


def _replay_band_colpass(bnd, widths, offs, M, x_stride, mode):
    """band_split.hip band_colpass_kernel: thread = 4 columns (V4, one band) or 1, block = 16 rows;
    reads x, inv (and g, dot); writes features (MODE 0) or dx and the partials (MODE 1)."""
    nb, F = len(widths), int(sum(widths))
    v4 = all(w % 4 == 0 for w in widths) and x_stride % 4 == 0
    C = 4 if v4 else 1
    blocks_x = cdiv(F, 256 * C)
    parts = cdiv(M, 16)
    t = np.arange(256)
    for bx in sorted({0, blocks_x - 1}):
        i = (bx * 256 + t) * C
        ok = i < F
        band = np.searchsorted(offs, np.minimum(i, F - 1), side="right") - 1
        if np.any(band[ok] < 0) or np.any(band[ok] >= nb):
            bnd.fail("colpass: band lookup out of range")
        bk = np.clip(band[ok], 0, nb - 1)
        if C == 4 and np.any((offs[bk + 1] < i[ok] + 4) | (offs[bk] > i[ok])):
            bnd.fail("colpass: a 4-column group crosses a band")
        bnd.touch("gamma", i * 4, 4 * C, ok)
        for by in sorted({0, parts - 1}):
            m0 = by * 16
            for r in sorted({0, min(16, M - m0) - 1}):
                m = m0 + r
                bnd.touch("x", (m * x_stride + i) * 4, 4 * C, ok)
                bnd.touch("inv_norm", (m * nb + np.clip(band, 0, nb - 1)) * 4, 4, ok)
                if mode == 0:
                    bnd.touch("features", (m * F + i) * 2, 2 * C, ok)
                else:
                    bnd.touch("g", (m * F + i) * 2, 2 * C, ok)
                    bnd.touch("dot", (m * nb + np.clip(band, 0, nb - 1)) * 4, 4, ok)
                    bnd.touch("dx", (m * F + i) * 4, 4 * C, ok)
            if mode == 1:
                bnd.touch("partial", (by * F + i) * 4, 4 * C, ok)


def replay_band_split_mixed(widths, M, O, *, x_stride=None):
    """band_split.hip launch_mixed_fwd / launch_mixed_bwd (the fp32-input band split, 16-bit projection):
    rowsum and column passes around the norm-free band GEMMs.  Yields (label, Bounds)."""
    nb, F = len(widths), int(sum(widths))
    offs = _offs(widths)
    x_stride = F if x_stride is None else x_stride
    fsizes = {"x": ((M - 1) * x_stride + F) * 4, "gamma": F * 4, "inv_norm": M * nb * 4, "features": M * F * 2,
              "offsets": (nb + 1) * 8}
    fwd = Bounds(dict(fsizes))
    _replay_band_rowsum(fwd, widths, offs, M, x_stride, 0, None)
    _replay_band_colpass(fwd, widths, offs, M, x_stride, 0)
    yield "band_split_mixed_fwd_norm", fwd
    # the norm-free GEMM on the 16-bit features (row pitch F)
    yield "band_split_mixed_fwd_gemm", replay_band_split_forward(widths, M, O, 2, norm=False)
    gb = cdiv(M * F * 2, 256) * 256
    db_ = cdiv(M * nb * 4, 256) * 256
    pb = cdiv(cdiv(M, 16) * F * 4, 256) * 256
    bsizes = {"x": ((M - 1) * x_stride + F) * 4, "gamma": F * 4, "inv_norm": M * nb * 4, "g": gb, "dot": db_,
              "partial": pb, "dx": M * F * 4, "dgamma": F * 4, "offsets": (nb + 1) * 8}
    bwd = Bounds(bsizes)
    _replay_band_rowsum(bwd, widths, offs, M, x_stride, 1, "g")
    _replay_band_colpass(bwd, widths, offs, M, x_stride, 1)
    _replay_col_sum(bwd, "partial", cdiv(M, 16), F, "dgamma", 4)
    yield "band_split_mixed_bwd_norm", bwd
    # g = T(dy W) on the norm-free dx kernel and dW / dbias on the norm-free register dW kernel: the
    # grouped-linear replay of those two kernels (dx = g here, x = the features)
    yield "band_split_mixed_bwd_gemm", replay_band_split_backward(widths, M, O, 2, grouped=True, even_dx=True)


GDX_TILES = {64: (4, 4, 4), 128: (8, 4, 4), 192: (12, 2, 4), 256: (16, 2, 4)}  # grouped_dx.hip launch_grouped_dx: DT, NT, stages
GDX_SLOTS = 2 * 256  # two blocks per CU on the 256 CUs of an MI355X


def gdx_tiles(I, G, M):
    """grouped_dx.hip launch_grouped_dx: (DT, NT, stages); at I = 192 the 48-row form when its block
    rounds x rows per wave are at most the 32-row form's."""
    if I != 192:
        return GDX_TILES[I]
    rounds = lambda rows: cdiv(G * cdiv(M, rows), GDX_SLOTS)  # noqa: E731
    return (12, 3, 3) if rounds(192) * 3 <= rounds(128) * 2 else GDX_TILES[192]


def gdx_row_tile(M, G, NT):
    """grouped_dx.hip launch_grouped_dx: the row tile (gdx_row_tile for the 48-row-wave form: the
    smallest multiple of 16 rows keeping the grid in the full tile's block rounds; the full 64 NT
    rows otherwise)."""
    full = 64 * NT
    if NT != 3:
        return full
    rounds = cdiv(G * cdiv(M, full), GDX_SLOTS)
    tiles = rounds * GDX_SLOTS // G
    if tiles <= 0:
        return full
    return min(full, cdiv(cdiv(M, tiles), 16) * 16)


def _replay_glin_dx(bnd, G, I, O, M, rb=None):
    """grouped_dx.hip glin_dx_kernel: the DMA ring of weight slabs and dy tiles, the transposed weight
    fragments, the dy B fragments and the dx stores, on the even block schedule."""
    DT, NT, S = gdx_tiles(I, G, M)
    kUnits, kSlab = I // 8, 32 * 2 * I
    kInstr = kSlab // 1024
    wave_rows = 16 * NT
    kStage = kSlab + 4 * wave_rows * 64
    bnd.sizes["lds_gdx"] = S * kStage
    if S * kStage > 160 * 1024:
        bnd.fail("glin_dx: more than 160 KB of LDS")
    if rb is None:
        rb = gdx_row_tile(M, G, NT)
    if rb % 16 or not 0 < rb <= 4 * wave_rows:
        bnd.fail("glin_dx: row tile not a multiple of 16 within the block's waves")
        return
    mtiles = cdiv(M, rb)
    units = lambda b: 1  # noqa: E731
    sc = build_even_sched(G, mtiles, units)
    decoded = sched_decode(sc, G, units, True, bnd, "glin_dx")
    lane = np.arange(64)
    gq, rr = lane >> 4, lane & 15
    nc = O // 32
    for g, mt, _ in sorted({(b, m, s_) for b, m, s_ in decoded if m in (0, mtiles - 1)}):
        for wave in range(4):
            npw = (kInstr - wave + 3) // 4
            for q in range(npw):
                t = wave + 4 * q
                P = 64 * t + lane
                kr, pu = P // kUnits, P % kUnits
                u = pu ^ swz_mn(kr)
                if np.any(u >= kUnits):
                    bnd.fail("glin_dx: swizzled unit leaves its row")
                for c in steps(nc):
                    bnd.touch("weight", g * O * I * 2 + ((32 * c + kr) * I + 8 * u) * 2, 16)
                for stage in range(S):
                    bnd.touch("lds_gdx", stage * kStage + t * 1024 + lane * 16, 16)
            wrow0 = mt * rb + wave * wave_rows
            left = min((mt + 1) * rb, M) - wrow0
            nvt = 0 if left <= 0 else (NT if left >= wave_rows else cdiv(left, 16))
            u = (lane & 3) ^ swz_k(lane >> 2)
            for n in range(nvt):
                m = np.minimum(wrow0 + 16 * n + (lane >> 2), M - 1)
                for c in steps(nc):
                    bnd.touch("dy", ((m * G + g) * O + 8 * u + 32 * c) * 2, 16)
                for stage in range(S):
                    bnd.touch("lds_gdx", stage * kStage + kSlab + (wave * NT + n) * 1024 + lane * 16, 16)
            if nvt == 0:
                continue
            jq = lane & 15
            kr0 = 8 * gq + (jq >> 2)
            for stage in range(S):
                base = stage * kStage
                for d in range(DT):
                    col = 16 * d + 4 * (jq & 3)
                    off = kr0 * 2 * I + 16 * ((col >> 3) ^ swz_mn(kr0)) + 2 * (col & 7)
                    bnd.touch("lds_gdx", base + off, 8)
                    bnd.touch("lds_gdx", base + off + 4 * 2 * I, 8)
                for n in range(NT):
                    bnd.touch("lds_gdx", base + kSlab + wave * NT * 1024 + rr * 64 + 16 * (gq ^ swz_k(rr)) + n * 1024, 16)
            for n in range(NT):
                m = wrow0 + 16 * n + rr
                ok = (n < nvt) & (m < M)
                for d in range(DT):
                    bnd.touch("dx", ((m * G + g) * I + 4 * gq + 16 * d) * 2, 8, ok)


def _replay_col_sum(bnd, pbuf, parts, dim, obuf, osz, poff=0):
    """rowgeom.h col_sum_tile (col_sum_kernel with 1024 threads, one row group each; the band-split DMA
    dW kernel's tail blocks with 256 threads, 4 groups each: the same rows): 64 row groups per 16
    columns, group g reading rows g, g + 64, ... (trips of 8 loads, then single loads); first and
    last tile."""
    tid = np.arange(256)
    cl, tg = tid % 16, tid // 16
    for blk in sorted({0, cdiv(dim, 16) - 1}):
        c = blk * 16 + cl
        ok = c < dim
        for v in range(4):
            p = tg + 16 * v
            while np.any(p + 7 * 64 < parts):
                live = p + 7 * 64 < parts
                for u in range(8):
                    bnd.touch(pbuf, poff + ((p + 64 * u) * dim + c) * 4, 4, ok & live)
                p = np.where(live, p + 8 * 64, p)
            while np.any(p < parts):
                bnd.touch(pbuf, poff + (p * dim + c) * 4, 4, ok & (p < parts))
                p = p + 64
        bnd.touch(obuf, c * osz, osz, ok & (tg == 0))


def _replay_bs_dw_dma(bnd, widths, offs, M, O, esz, has_bias):
    """band_split.hip bs_bwd_dw_dma_kernel (S = 3 stages, KS = 2: 64 rows per step)."""
    S, KS = 3, 2
    KR = KS * CHUNK_K
    kTile = KR * 2 * 64
    kStage = 2 * kTile
    kWR = KR // 4
    kXI, kDI = kWR // 2, kWR // 8
    nb, F = len(widths), int(sum(widths))
    otiles = cdiv(O, 64)
    units = lambda b: cdiv(widths[b], 64) * otiles  # noqa: E731
    sc = build_band_sched(nb, 1, units)
    if sc is None:
        bnd.fail("dw dma: no schedule")
        return
    bnd.sizes["lds"] = max(bnd.sizes["lds"], S * kStage + 2048 * 4)
    decoded = sched_decode(sc, nb, units, False, bnd, "bs_bwd_dw_dma")
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    wr, wc = wave >> 1, wave & 1
    nk = cdiv(M, KR)
    kbeg = M - nk * KR
    dstride = nb * O
    for band, _mt, sub in sorted(set(decoded)):
        i0, o0 = sub // otiles * 64, sub % otiles * 64
        off, I = int(offs[band]), int(widths[band])
        for c in steps(nk):
            stage = (c % S) * kStage
            for t in range(kDI):
                r = kWR * wave + 8 * t + (lane >> 3)
                col = np.minimum(o0 + 8 * ((lane & 7) ^ swz_mn(r)), O - 8)
                row = kbeg + c * KR + r
                row = np.where((c == 0) & (row < 0), 0, row)
                bnd.touch("dy", (row * dstride + band * O + col) * esz, 16)
                bnd.touch("lds", stage + kTile + 128 * (kWR * wave + 8 * t) + 16 * lane, 16)
            for t in range(kXI):
                r = kWR * wave + 2 * t + (lane >> 5)
                i = np.minimum(i0 + 8 * (((lane & 31) >> 2) ^ swz_mn(r)) + 2 * (lane & 3), I - 2)
                row = kbeg + c * KR + r
                row = np.where((c == 0) & (row < 0), 0, row)
                bnd.touch("x", (row * F + off + i) * esz, 4)
                bnd.touch("lds", stage + 128 * (kWR * wave + 2 * t) + 4 * lane, 4)
            # inv window, scaling pass and fragment reads
            urow = kWR * wave + (lane >> 3)
            uoff = urow * 2 * 64 + 16 * (lane & 7)
            for j in range(KS):
                bnd.touch("lds", stage + uoff + 8 * j * 128, 16)
            for kk in range(KS):
                for f in range(2):
                    fa = frag_mn_addr(0, 32 * wr + 16 * f, 2 * 64, lane) + stage + kk * 32 * 128
                    fb = frag_mn_addr(kTile, 32 * wc + 16 * f, 2 * 64, lane) + stage + kk * 32 * 128
                    for a in (fa, fb):
                        bnd.touch("lds", a, 8)
                        bnd.touch("lds", a + 4 * 2 * 64, 8)
        for c0 in range(0, nk, 2048 // KR):
            j = np.arange(min((nk - c0) * KR, 2048))
            rr = kbeg + c0 * KR + j
            bnd.touch("inv_norm", (rr * nb + band) * 4, 4, rr >= 0)
        for f in range(2):
            i = i0 + 32 * wr + 16 * f + 4 * (lane >> 4)
            for r in range(4):
                bnd.touch("gamma", (off + np.minimum(i + r, I - 1)) * esz, esz)
        if has_bias and i0 == 0:
            for g in range(2):
                o = o0 + 32 * wc + 16 * g + lane
                bnd.touch("db", (band * O + o) * esz, esz, (wr == 0) & (lane < 16) & (o < O))
        kop = 64 + 8
        for f in range(2):
            for g in range(2):
                bnd.touch("lds", ((32 * wc + 16 * g + (lane & 15)) * kop + 32 * wr + 16 * f + 4 * (lane >> 4)) * esz,
                          4 * esz)
        iv = min(I - i0, 64)
        q = tid & 15
        for p in range(4):
            ol = (tid >> 4) + 16 * p
            ok = (o0 + ol < O) & (4 * q < iv)
            bnd.touch("lds", (ol * kop + 4 * q) * esz, 8, ok)
            bnd.touch("dw", (O * off + (o0 + ol) * I + i0 + 4 * q) * esz, 8, ok)


def _replay_bs_dw_reg(bnd, widths, offs, M, O, esz, has_bias, norm, v4):
    """band_split.hip bs_bwd_dw_kernel (register-staged main loop; also the grouped linear's dW)."""
    nb, F = len(widths), int(sum(widths))
    max_it = cdiv(max(widths), 64)
    # the even schedule over the existing (band, input tile, output tile) blocks (sub = input tile x
    # output tiles + output tile); the XcdGrid past 256 bands
    otiles = cdiv(O, 64)
    units = lambda b: cdiv(widths[b], 64) * otiles
    sc = build_even_sched(nb, 1, units)
    if sc is not None:
        dec = sched_decode(sc, nb, units, False, bnd, "bs_bwd_dw")
        blocks = [(b * max_it + sub // otiles, sub % otiles) for b, _, sub in dec]
    else:
        grp, ot, valid = xcd_decode(nb * max_it, otiles)
        blocks = list(zip(grp[valid], ot[valid]))
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    nk = cdiv(M, CHUNK_K)
    kbeg = M - nk * CHUNK_K
    bnd.sizes["lds"] = max(bnd.sizes["lds"], gemm_lds_bytes(esz, 64, 64))
    for g_, o_ in blocks:
        band, i0 = int(g_) // max_it, (int(g_) % max_it) * 64
        o0 = int(o_) * 64
        off, I = int(offs[band]), int(widths[band])
        if i0 >= I or M == 0:
            continue
        mn_loader(bnd, "x", esz, off + i0, F, I - i0, M, 64, v4, kbeg, nk, tid)
        if norm:
            bnd.touch("inv_norm", (np.arange(M) * nb + band) * 4, 4)
        mn_loader(bnd, "dy", esz, band * O + o0, nb * O, O - o0, M, 64, v4, kbeg, nk, tid)
        if has_bias and i0 == 0:
            t64 = np.arange(GEMM_THREADS)
            bnd.touch("db", (band * O + o0 + t64) * esz, esz, (t64 < 64) & (t64 < O - o0))
        ir, oc = (wave >> 1) * 32, (wave & 1) * 32
        for u in range(2):
            i = i0 + ir + u * 16 + 4 * (lane >> 4)
            for v in range(2):
                o = o0 + oc + v * 16 + (lane & 15)
                ok = (i < I) & (o < O)
                if v4:
                    bnd.touch("dw", (O * off + o * I + i) * esz, 4 * esz, ok)
                else:
                    for r in range(4):
                        bnd.touch("dw", (O * off + o * I + i + r) * esz, esz, ok & (i + r < I))


# ----------------------------------------------------------------------------- mask estimator


def replay_mask_final_forward(widths, M, H, esz):
    """mask_estimator.hip launch_me_fwd: me_fwd_dma_kernel on the band schedule (16-bit, aligned), else
    me_fwd_kernel."""
    nb, F = len(widths), int(sum(widths))
    offs = _offs(widths)
    sizes = {"x": M * nb * H * esz, "weight": 2 * F * H * esz, "bias": 2 * F * esz, "pre": M * 2 * F * esz,
             "out": M * F * esz, "offsets": (nb + 1) * 8, "lds": 4 * 16384}
    bnd = Bounds(sizes)
    vec4 = all(w % 4 == 0 for w in widths) and H % 4 == 0
    mtiles = cdiv(M, 128)
    if not (esz == 2 and vec4 and H % 8 == 0 and H > CHUNK_K):
        _replay_me_fwd_reg(bnd, widths, offs, M, H, esz, vec4)
        return bnd
    units = lambda b: cdiv(widths[b], 64)  # noqa: E731
    sc = build_band_sched(nb, mtiles, units)
    decoded = sched_decode(sc, nb, units, False, bnd, "me_fwd_dma")
    S, kStage = 4, 16384
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    g, rr = lane >> 4, lane & 15
    wr, wc = wave >> 1, wave & 1
    u = (lane & 3) ^ swz_k(lane >> 2)
    rsub = lane >> 2
    nk = cdiv(H, CHUNK_K)
    kbeg = H - nk * CHUNK_K
    for band, mt, chunk in sorted({(b, m, s) for b, m, s in decoded if m in (0, mtiles - 1)}):
        l0 = chunk * 64
        off, I = int(offs[band]), int(widths[band])
        m0 = mt * 128
        rv = min(M - m0, 128)
        active = l0 + 32 * wr < I
        nv = np.where(wave >= 2, 4, np.where(l0 + 32 * wave + 16 < I, 4, np.where(l0 + 32 * wave < I, 2, 0)))
        for t in range(4):
            R = 64 * wave + 16 * t + rsub
            l = l0 + 16 * (R >> 5) + (R & 15)
            lc = np.minimum(l, I - 1)
            wrow = np.where(((R >> 4) & 1) == 1, I + lc, lc)
            m = np.minimum(R - 128, rv - 1)
            is_w = wave < 2
            gb_w = 2 * off * H
            gb_x = (m0 * nb + band) * H
            # chunk 0 through registers: units with k < 0 read k = 0 of the row
            ok0 = kbeg + 8 * u >= 0
            kel = np.where(ok0, kbeg + 8 * u, 0)
            bnd.touch("weight", (gb_w + wrow * H + kel) * esz, 16, is_w)
            bnd.touch("x", (gb_x + m * nb * H + kel) * esz, 16, ~is_w)
            bnd.touch("lds", 4 * wave * 1024 + t * 1024 + lane * 16, 16)
            for c in steps(nk):
                if c == 0:
                    continue
                cc = min(c, nk - 1)
                k = kbeg + CHUNK_K * cc + 8 * u
                live = t < nv
                bnd.touch("weight", (gb_w + wrow * H + k) * esz, 16, is_w & live)
                bnd.touch("x", (gb_x + m * nb * H + k) * esz, 16, (~is_w) & live)
                bnd.touch("lds", 4 * wave * 1024 + (cc % S) * kStage + t * 1024 + lane * 16, 16, live)
        sw = 16 * (g ^ swz_k(rr))
        for st in {0, (S - 1) * kStage}:
            for q in range(4):
                bnd.touch("lds", (64 * wr + rr) * 64 + sw + st + 1024 * q, 16, active)
                bnd.touch("lds", 8192 + (64 * wc + rr) * 64 + sw + st + 1024 * q, 16, active)
        kop = 72
        for h in range(2):
            lt = 32 * wr + 16 * h + 4 * g
            l = l0 + lt
            okl = active & (l < I)
            bnd.touch("bias", (2 * off + l) * esz, 4 * esz, okl)
            bnd.touch("bias", (2 * off + I + l) * esz, 4 * esz, okl)
            for j in range(4):
                m = 64 * wc + 16 * j + rr
                for base in (0, 128 * kop, 2 * 128 * kop):
                    bnd.touch("lds", (base + m * kop + lt) * esz, 4 * esz, active)
        c4 = (tid & 15) * 4
        for p in range(8):
            m = (tid >> 4) + 16 * p
            ok = (l0 + c4 < I) & (m < rv)
            bnd.touch("pre", ((m0 + m) * 2 * F + 2 * off + l0 + c4) * esz, 8, ok)
            bnd.touch("pre", ((m0 + m) * 2 * F + 2 * off + l0 + c4 + I) * esz, 8, ok)
            bnd.touch("out", ((m0 + m) * F + off + l0 + c4) * esz, 8, ok)
    bnd.touch("offsets", np.arange(nb + 1) * 8, 8)
    return bnd


DW_CUS = 256        # CUs of the device the dW tile choice is replayed for
LDS_PER_CU = 160 * 1024


def dw_jt(groups, in_features, out_features):
    """mask_estimator.hip launch_uniform_dw_impl: the j tile (192 when it takes fewer rounds of
    resident blocks than 128, with rings of 3 stages of 32 K-rows x (64 + JT) columns)."""
    htl = in_features // 64

    def rounds(jt):
        ring = 3 * CHUNK_K * 2 * (64 + jt)
        return cdiv(groups * htl * cdiv(out_features, jt), DW_CUS * (LDS_PER_CU // ring))

    return 192 if rounds(192) < rounds(128) else 128


def _replay_me_dw_dma(bnd, widths, offs, M, H, esz, HT, dpre_buf, x_buf, dw_buf, db_buf, lds_buf, JT=128):
    """mask_estimator.hip me_bwd_dw_dma_kernel<T, HT, JT> (HT hidden columns x JT j per block,
    (HT / 64) x (JT / 64) waves, the x and dpre tiles moved as one list of 1 KB pieces dealt to the
    waves in turn) on its band schedule, over a dpre-like buffer of row pitch 2 F."""
    nb, F = len(widths), int(sum(widths))
    S2 = 3
    WJ = JT // 64
    NW2 = HT // 64 * WJ
    kU2, kJU = HT // 8, JT // 8
    kXTile = CHUNK_K * HT * 2
    kStage2 = kXTile + CHUNK_K * JT * 2
    PX = kXTile // 1024
    PT = PX + CHUNK_K * JT * 2 // 1024
    kMaxPW = cdiv(PT, NW2)
    bnd.sizes[lds_buf] = max(bnd.sizes.get(lds_buf, 0), S2 * kStage2)
    htl = H // HT
    units2 = lambda b: htl * cdiv(2 * widths[b], JT)  # noqa: E731
    sc2 = build_band_sched(nb, 1, units2)
    decoded2 = sched_decode(sc2, nb, units2, False, bnd, "me_bwd_dw_dma")
    tid = np.arange(NW2 * 64)
    lane, wave = tid & 63, tid >> 6
    wr, wc = wave // WJ, wave % WJ
    nk = cdiv(M, CHUNK_K)
    kbeg = M - nk * CHUNK_K
    xstride = nb * H
    for band, _mt, sub in sorted(set(decoded2)):
        off, I = int(offs[band]), int(widths[band])
        K2 = 2 * I
        h0 = (sub % htl) * HT
        j0 = (sub // htl) * JT
        for c in steps(nk):
            st = (c % S2) * kStage2
            for t in range(kMaxPW):
                k = wave + NW2 * t
                valid = k < PT
                isx = k < PX
                units = np.where(isx, kU2, kJU)
                U = 64 * np.where(isx, k, k - PX) + lane
                kr = U // units
                uu = (U % units) ^ swz_mn(kr)
                row = kbeg + c * CHUNK_K + kr
                row = np.where((c == 0) & (row < 0), 0, row)
                bnd.touch(x_buf, (row * xstride + band * H + h0 + 8 * uu) * esz, 16, valid & isx)
                jc = np.minimum(j0 + 8 * uu, K2 - 8)
                bnd.touch(dpre_buf, (row * 2 * F + 2 * off + jc) * esz, 16, valid & ~isx)
                bnd.touch(lds_buf, st + k * 1024 + 16 * lane, 16, valid)
            for i in range(4):
                fa = frag_mn_addr(0, 64 * wr + 16 * i, 2 * HT, lane) + st
                fb = frag_mn_addr(kXTile, 64 * wc + 16 * i, 2 * JT, lane) + st
                for a_, p in ((fa, 2 * HT), (fb, 2 * JT)):
                    bnd.touch(lds_buf, a_, 8)
                    bnd.touch(lds_buf, a_ + 4 * p, 8)
        jv = min(K2 - j0, JT)
        if db_buf is not None:
            for j in range(4):
                jj = 64 * wc + 16 * j + lane
                bnd.touch(db_buf, (2 * off + j0 + jj) * esz, esz, (h0 == 0) & (wr == 0) & (lane < 16) & (jj < jv))
        kop = HT + 8
        if JT * kop * 2 > S2 * kStage2:
            bnd.fail("me_bwd_dw_dma: staging tile larger than the ring")
        for j in range(4):
            jj = 64 * wc + 16 * j + (lane & 15)
            for i in range(4):
                bnd.touch(lds_buf, (jj * kop + 64 * wr + 16 * i + 4 * (lane >> 4)) * esz, 4 * esz)
        rows_per_pass = 64 * NW2 // kU2
        c8 = (tid % kU2) * 8
        for p in range(JT // rows_per_pass):
            jj = tid // kU2 + rows_per_pass * p
            ok = jj < jv
            bnd.touch(lds_buf, (jj * kop + c8) * esz, 16, ok)
            bnd.touch(dw_buf, ((2 * off + j0 + jj) * H + h0 + c8) * esz, 16, ok)


def _replay_me_dz(bnd, widths, offs, M, H, esz, tanh_in):
    """mask_dz.hip me_dz_kernel: the ring of weight slabs (rows clamped to the band) and dpre tiles
    (columns clamped to the band), the transposed weight fragments, the dpre B fragments, the x
    prefetch (tanh input) and the dz stores, on the cost-balanced band schedule."""
    nb, F = len(widths), int(sum(widths))
    DT, NT = (12, 2) if H % 192 == 0 else (8, 2)
    S, HT = 4, 16 * DT
    kUnits, kSlab = HT // 8, 32 * 2 * HT
    kInstr = kSlab // 1024
    wave_rows = 16 * NT
    kStage = kSlab + 4 * wave_rows * 64
    bnd.sizes["lds_dz"] = S * kStage
    if S * kStage > 160 * 1024:
        bnd.fail("me_dz: more than 160 KB of LDS")
    mtiles = cdiv(M, 4 * wave_rows)
    units = lambda b: H // HT  # noqa: E731
    sc = build_band_sched(nb, mtiles, units, lambda b: cdiv(2 * widths[b], 32) + 5)
    decoded = sched_decode(sc, nb, units, True, bnd, "me_dz")
    lane = np.arange(64)
    gq, rr = lane >> 4, lane & 15
    for band, mt, sub in sorted({(b, m, s_) for b, m, s_ in decoded if m in (0, mtiles - 1)}):
        off, I = int(offs[band]), int(widths[band])
        K = 2 * I
        nc = cdiv(K, 32)
        h0 = sub * HT
        for wave in range(4):
            wrow0 = mt * 4 * wave_rows + wave * wave_rows
            left = M - wrow0
            nvt = 0 if left <= 0 else (NT if left >= wave_rows else cdiv(left, 16))
            npw = (kInstr - wave + 3) // 4
            for q in range(npw):
                t = wave + 4 * q
                P = 64 * t + lane
                kr, pu = P // kUnits, P % kUnits
                col = h0 + 8 * (pu ^ swz_mn(kr))
                if np.any(pu ^ swz_mn(kr) >= kUnits):
                    bnd.fail("me_dz: swizzled unit leaves its row")
                for c in steps(nc):
                    j = np.minimum(32 * c + kr, K - 1)
                    bnd.touch("weight", ((2 * off + j) * H + col) * esz, 16)
                for stage in range(S):
                    bnd.touch("lds_dz", stage * kStage + t * 1024 + lane * 16, 16)
            du = (lane & 3) ^ swz_k(lane >> 2)
            for n in range(nvt):
                m = np.minimum(wrow0 + 16 * n + (lane >> 2), M - 1)
                for c in steps(nc):
                    col = np.minimum(32 * c + 8 * du, K - 8)
                    bnd.touch("workspace", (m * 2 * F + 2 * off + col) * esz, 16)
                for stage in range(S):
                    bnd.touch("lds_dz", stage * kStage + kSlab + (wave * NT + n) * 1024 + lane * 16, 16)
            if nvt == 0:
                continue
            jq = lane & 15
            kr0 = 8 * gq + (jq >> 2)
            for stage in range(S):
                base = stage * kStage
                for d in range(DT):
                    col = 16 * d + 4 * (jq & 3)
                    o = kr0 * 2 * HT + 16 * ((col >> 3) ^ swz_mn(kr0)) + 2 * (col & 7)
                    bnd.touch("lds_dz", base + o, 8)
                    bnd.touch("lds_dz", base + o + 4 * 2 * HT, 8)
                for n in range(NT):
                    bnd.touch("lds_dz", base + kSlab + wave * NT * 1024 + rr * 64 + 16 * (gq ^ swz_k(rr)) + n * 1024, 16)
            kop = HT + 8
            for n in range(NT):  # staging writes of the epilogue
                r = wave * wave_rows + 16 * n + rr
                for d in range(DT):
                    bnd.touch("lds_dz", (r * kop + 16 * d + 4 * gq) * esz, 4 * esz)
        # epilogue: 16-byte units along whole rows (x read with clamped rows, dx written for m < M)
        kop = HT + 8
        if 4 * wave_rows * kop * esz > S * kStage:
            bnd.fail("me_dz: staging tile larger than the ring")
        tid = np.arange(256)
        m0 = mt * 4 * wave_rows
        for k in range(4 * wave_rows * kUnits // 256):
            q = tid + 256 * k
            r, u = q // kUnits, q % kUnits
            if tanh_in:
                m = np.minimum(m0 + r, M - 1)
                bnd.touch("x", ((m * nb + band) * H + h0 + 8 * u) * esz, 16)
            ok = m0 + r < M
            bnd.touch("lds_dz", (r * kop + 8 * u) * esz, 16, ok)
            bnd.touch("dx", (((m0 + r) * nb + band) * H + h0 + 8 * u) * esz, 16, ok)


def replay_mask_final_backward(widths, M, H, esz, *, tanh_in=False):
    """mask_estimator.hip launch_me_bwd: me_dpre_flat_kernel, me_bwd_dx_dma_kernel (HC = 256 when
    H % 256 == 0, else 128), me_bwd_dw_dma_kernel (HT = 128)."""
    nb, F = len(widths), int(sum(widths))
    offs = _offs(widths)
    sizes = {"gout": M * F * esz, "x": M * nb * H * esz, "pre": M * 2 * F * esz, "weight": 2 * F * H * esz,
             "dx": M * nb * H * esz, "dbias": 2 * F * esz, "dw": 2 * F * H * esz,
             "workspace": cdiv(M * 2 * F * esz, 256) * 256, "offsets": (nb + 1) * 8, "lds": 0,
             "lds_flat": (4096 + 1) * 4}
    bnd = Bounds(sizes)
    vec4 = all(w % 4 == 0 for w in widths) and H % 4 == 0
    if not vec4:
        bnd.fail("mask backward: unaligned widths not modelled")
        return bnd
    dz_ring = esz == 2 and (H % 192 == 0 or H % 128 == 0)  # mask_dz.hip me_dz_kernel
    dma_dx = esz == 2 and H % 128 == 0 and not dz_ring
    dma_dw = esz == 2 and M >= CHUNK_K and H % 128 == 0
    # -- dpre over whole rows: 4 columns per thread
    V = 4
    nq = F // V
    rows = 4  # kDpreFlatRows
    flat_threads = cdiv(M, rows) * nq
    if flat_threads + 255 >= 1 << 31:
        bnd.fail("dpre: thread index past 32 bits")
    nblk = cdiv(flat_threads, 256)
    tid = np.arange(256)
    for blk in sorted({0, 1, nblk - 1}):
        t = blk * 256 + tid
        m0 = t // nq * rows
        live = m0 < M
        c0 = V * (t % nq)
        band = np.searchsorted(offs[:-1], c0, side="right") - 1
        off = offs[band]
        I = offs[band + 1] - off
        l = c0 - off
        if np.any(l + V > I):
            bnd.fail("dpre: a column group crosses a band")
        for r in range(rows):
            m = np.minimum(m0 + r, M - 1)
            bnd.touch("gout", (m * F + c0) * esz, V * esz, live)
            bnd.touch("pre", (m * 2 * F + 2 * off + l) * esz, V * esz, live)
            bnd.touch("pre", (m * 2 * F + 2 * off + l + I) * esz, V * esz, live)
            okw = live & (m0 + r < M)
            bnd.touch("workspace", ((m0 + r) * 2 * F + 2 * off + l) * esz, V * esz, okw)
            bnd.touch("workspace", ((m0 + r) * 2 * F + 2 * off + l + I) * esz, V * esz, okw)
    bnd.touch("lds_flat", np.arange(nb + 1) * 4, 4)
    if dz_ring:
        _replay_me_dz(bnd, widths, offs, M, H, esz, tanh_in)
    elif not dma_dx:
        _replay_me_dx_reg(bnd, widths, offs, M, H, esz, tanh_in)
    if not dma_dw:
        _replay_me_dw_reg(bnd, widths, offs, M, H, esz)
    if not (dma_dx or dma_dw):
        bnd.touch("offsets", np.arange(nb + 1) * 8, 8)
        return bnd
    # -- dx on the DMA ring
    HC = 256 if H % 256 == 0 else 128
    S = 3 if HC == 256 else 4
    NW = HC // 32
    kU = HC // 8
    kWTile = CHUNK_K * HC * 2
    kStage = kWTile + 8192
    kDI = 8 // NW
    bnd.sizes["lds"] = S * kStage
    nhc = H // HC
    mt_dx = cdiv(M, 128)
    units = lambda b: nhc  # noqa: E731
    sc = build_band_sched(nb, mt_dx, units, lambda b: cdiv(2 * widths[b], CHUNK_K) + 2)
    decoded = sched_decode(sc, nb, units, True, bnd, "me_bwd_dx_dma")
    tid = np.arange(NW * 64)
    lane, wave = tid & 63, tid >> 6
    wr, wc = wave >> 1, wave & 1
    for band, mt, hc in sorted({(b, m, s) for b, m, s in decoded if m in (0, mt_dx - 1) and dma_dx}):
        off, I = int(offs[band]), int(widths[band])
        K = 2 * I
        m0 = mt * 128
        rv = min(M - m0, 128)
        nk = cdiv(K, CHUNK_K)
        kbeg = K - nk * CHUNK_K
        ub = (lane & 3) ^ swz_k((lane >> 2) & 15)
        bok0 = kbeg + 8 * ub >= 0
        for c in steps(nk):
            st = (c % S) * kStage
            for t in range(2):
                kr = (64 // kU) * (wave + NW * t) + lane // kU
                ua = (lane % kU) ^ swz_mn_p(2 * HC, kr)
                row = kbeg + c * CHUNK_K + kr
                row = np.where((c == 0) & (row < 0), 0, row)
                bnd.touch("weight", ((2 * off + row) * H + hc * HC + 8 * ua) * esz, 16)
                bnd.touch("lds", st + (wave + NW * t) * 1024 + 16 * lane, 16)
            for t in range(kDI):
                mr = 16 * (wave + NW * t) + (lane >> 2)
                mrc = np.minimum(mr, rv - 1)
                col = kbeg + c * CHUNK_K + 8 * ub
                col = np.where((c == 0) & ~bok0, 0, col)
                bnd.touch("workspace", ((m0 + mrc) * 2 * F + 2 * off + col) * esz, 16)
                bnd.touch("lds", st + kWTile + (wave + NW * t) * 1024 + 16 * lane, 16)
            for i in range(4):
                fa = frag_mn_addr(0, 64 * wr + 16 * i, 2 * HC, lane, p512=True) + st
                bnd.touch("lds", fa, 8)
                bnd.touch("lds", fa + 4 * 2 * HC, 8)
            fb = frag_k_addr(kWTile, 64 * wc, lane) + st
            for j in range(4):
                bnd.touch("lds", fb + 1024 * j, 16)
        kop = HC + 8
        for j in range(4):
            m = 64 * wc + 16 * j + (lane & 15)
            for i in range(4):
                h = 64 * wr + 16 * i + 4 * (lane >> 4)
                if tanh_in:
                    mc = np.minimum(m, rv - 1)
                    bnd.touch("x", (((m0 + mc) * nb + band) * H + hc * HC + h) * esz, 4 * esz)
                bnd.touch("lds", (m * kop + h) * esz, 4 * esz)
        c8 = (tid % kU) * 8
        for p in range(128 // 16):
            row = tid // kU + 16 * p
            ok = row < rv
            bnd.touch("lds", (row * kop + c8) * esz, 16, ok)
            bnd.touch("dx", (((m0 + row) * nb + band) * H + hc * HC + c8) * esz, 16, ok)
    # -- dW on the DMA ring
    if dma_dw:
        _replay_me_dw_dma(bnd, widths, offs, M, H, esz, 128, "workspace", "x", "dw", "dbias", "lds")
    bnd.touch("offsets", np.arange(nb + 1) * 8, 8)
    return bnd


MLP_TILES = {64: (2, 4, 4), 128: (4, 4, 4), 192: (6, 2, 8), 256: (8, 4, 4), 384: (12, 2, 4), 512: (16, 2, 4)}


def mlp_row_tile(M, NT, WV):
    """mask_mlp.hip mlp_row_tile: the rows of a block's row tile (full - 32 where the full tile would
    leave at most an eighth of itself in the last tile and full - 32 needs no extra tile)."""
    full = 16 * NT * WV
    tiles = cdiv(M, full)
    tail = M - (tiles - 1) * full
    alt = full - 32
    if M > full and tail <= full // 8 and cdiv(M, alt) == tiles:
        return alt
    return full


def replay_mask_mlp_forward(widths, M, D, H, esz, *, write_h=True, wv=None, apply=None, rb=None):
    """mask_mlp.hip mlp_fwd_kernel (whole depth-2 mask MLP, 16-bit) on its band schedule: the b1 fill,
    the x fragments, the W1 / W2 DMA ring, the LDS fragment reads, the hidden stores and the GLU
    epilogue."""
    nb, F = len(widths), int(sum(widths))
    offs = _offs(widths)
    DK, NT, WV = MLP_TILES[D]
    if wv is not None:  # same rows per block
        NT, WV = NT * WV // wv, wv
    S, J = (2 if DK >= 12 else 3), 64
    kStage = DK * 2048 + 2 * J * 64
    sizes = {"x": M * nb * D * esz, "w1": nb * H * D * esz, "b1": nb * H * esz, "w2": 2 * F * H * esz,
             "b2": 2 * F * esz, "pre": M * 2 * F * esz, "out": M * F * esz, "hid": M * nb * H * esz,
             "offsets": (nb + 1) * 8, "lds": S * kStage, "sb1": 2048 * 4, "tanh": 2 * 32768 * 2,
             "stab": 32768 * 2}
    if apply is not None:
        if M % apply["frames"] or F % (2 * apply["channels"]):
            raise ValueError("apply: rows must be batch * frames and features 2 * channels * bins")
        bsz = M // apply["frames"]
        sizes["spec"] = bsz * (F // 2) * apply["frames"] * 8
        sizes["est"] = bsz * apply["stems"] * (F // 2) * apply["frames"] * 8
    bnd = Bounds(sizes)
    if S * kStage + 32768 * 2 + 2048 * 4 > 160 * 1024:
        bnd.fail("mlp_fwd: more than 160 KB of LDS")
    if H > 2048 or H % 32 or any(w % 4 for w in widths):
        bnd.fail("mask_mlp: shape outside the host check")
        return bnd
    wave_rows = 16 * NT
    if rb is None:
        rb = mlp_row_tile(M, NT, WV)
    if rb % 16 or not 0 < rb <= WV * wave_rows:
        bnd.fail("mlp_fwd: row tile not a multiple of 16 within the block's waves")
        return bnd
    mtiles = cdiv(M, rb)
    units = lambda b: cdiv(widths[b], J)  # noqa: E731

    def nv_of(b, p):  # the kernel's instance: 1, 2 or 4 16-row output groups per half
        groups = cdiv(widths[b] - J * p, 16)
        return 4 if groups >= 3 else groups

    sc = build_even_sched(nb, mtiles, units)
    decoded = sched_decode(sc, nb, units, True, bnd, "mlp_fwd")
    tid = np.arange(64 * WV)
    lane = tid & 63
    g, rr = lane >> 4, lane & 15
    u = (lane & 3) ^ swz_k(lane >> 2)
    nc = H // 32
    for band, mt, pss in sorted({(b, m, p) for b, m, p in decoded if m in (0, mtiles - 1)}):
        off, I = int(offs[band]), int(widths[band])
        j0 = pss * J
        NV = nv_of(band, pss)
        kmax_pw = (2 * DK + 2 * NV + WV - 1) // WV
        for i0 in range(0, H, 64 * WV):
            i = i0 + tid
            bnd.touch("b1", (band * H + i) * esz, esz, i < H)
            bnd.touch("sb1", i * 4, 4, i < H)
        for k in range(64):  # tanh table: 64 DMAs of 1 KB (wave k % WV), bf16 table first
            bnd.touch("tanh", k * 1024 + lane * 16, 16)
            bnd.touch("stab", k * 1024 + lane * 16, 16)
        bnd.touch("stab", np.array([0, 0x7FFF]) * 2, 2)  # table reads: index = pattern & 0x7fff
        nv2 = min(NV, cdiv(I - j0, 16))
        ntot = 2 * DK + 2 * nv2
        if WV > 2 * DK:
            bnd.fail("mlp_fwd: a wave's padding DMA would not repeat a W1 piece")
        for wave in range(WV):
            npw = (ntot - wave + WV - 1) // WV
            if npw > kmax_pw:
                bnd.fail("mlp_fwd: more DMA instructions than the plan holds")
            # with padding (all but dim 256) every wave issues kmax_pw DMAs, those past its share
            # repeating piece k = wave
            pad = DK != 8  # kLean
            for q in range(kmax_pw if pad else npw):
                k = wave + WV * q if q < npw else wave
                if k < 2 * DK:
                    r = 16 * (k & 1) + (lane >> 2)
                    gsrc = (r * D + 32 * (k >> 1) + 8 * u) * 2
                    ldst = (k >> 1) * 2048 + (k & 1) * 1024
                    base, stride, buf = band * H * D * esz, 64 * D, "w1"
                else:
                    k2 = k - 2 * DK
                    half, grp = k2 // nv2, k2 % nv2
                    jr = j0 + 16 * grp + (lane >> 2)
                    jc = np.minimum(jr, I - 1)
                    prow = I + jc if half else jc
                    gsrc = (prow * H + 8 * u) * 2
                    ldst = DK * 2048 + (4 * half + grp) * 1024
                    base, stride, buf = 2 * off * H * esz, 64, "w2"
                    if ldst + 1024 > kStage:
                        bnd.fail("mlp_fwd: W2 group outside the stage")
                if np.any(gsrc + (nc - 1) * stride >= 1 << 32):
                    bnd.fail("mlp_fwd: 32-bit DMA offset overflows")
                for c in steps(nc):
                    bnd.touch(buf, base + gsrc + c * stride, 16)
                for stage in range(S):
                    bnd.touch("lds", stage * kStage + ldst + lane * 16, 16)
            wrow0 = mt * rb + wave * wave_rows
            left = min((mt + 1) * rb, M) - wrow0
            nvt = 0 if left <= 0 else (NT if left >= wave_rows else cdiv(left, 16))
            for n in range(NT):
                m = np.minimum(wrow0 + 16 * n + rr, M - 1)
                for s_ in range(DK):
                    bnd.touch("x", ((m * nb + band) * D + 8 * g + 32 * s_) * esz, 16)
            if nvt == 0:
                continue
            for stage in range(S):
                sb = stage * kStage
                for t in range(2):
                    r = 8 * (rr >> 2) + 4 * t + (rr & 3)
                    a1 = r * 64 + 16 * (g ^ swz_k(r & 15))
                    for s_ in range(DK):
                        bnd.touch("lds", sb + a1 + 2048 * s_, 16)
                a2 = DK * 2048 + rr * 64 + 16 * (g ^ swz_k(rr))
                for t in range(2 * NV):  # the instance's 2 NV GEMM2 row tiles (W2 groups t, 4 + t)
                    bnd.touch("lds", sb + a2 + 1024 * (t if t < NV else 4 + t - NV), 16)
            for c in steps(nc):
                bnd.touch("sb1", (32 * c + 8 * g) * 4, 32)
                if write_h:
                    for n in range(NT):
                        m = wrow0 + 16 * n + rr
                        bnd.touch("hid", ((m * nb + band) * H + 32 * c + 8 * g) * esz, 16, (n < nvt) & (m < M))
            # epilogue loads first, from addresses clamped into the band (and rows, for the spectrum)
            for t in range(NV):
                jt = j0 + 16 * t + 4 * g
                jc = np.where((t < nv2) & (jt < I), jt, I - 4)
                bnd.touch("b2", (2 * off + jc) * esz, 4 * esz)
                bnd.touch("b2", (2 * off + I + jc) * esz, 4 * esz)
                if apply is not None:
                    fr, ch = apply["frames"], apply["channels"]
                    fbins = F // (2 * ch)
                    for n in range(NT):
                        mm = np.minimum(wrow0 + 16 * n + rr, M - 1)
                        bb, tt = mm // fr, mm % fr
                        for q in range(2):
                            r = (off + jc) // 2 + q
                            bnd.touch("spec", ((bb * fbins * ch + r) * fr + tt) * 8, 8)
            for t in range(NV):
                j = j0 + 16 * t + 4 * g
                okj = (t < nv2) & (j < I)
                for n in range(NT):
                    m = wrow0 + 16 * n + rr
                    ok = okj & (n < nvt) & (m < M)
                    bnd.touch("pre", (m * 2 * F + 2 * off + j) * esz, 4 * esz, ok)
                    bnd.touch("pre", (m * 2 * F + 2 * off + I + j) * esz, 4 * esz, ok)
                    if apply is None:
                        bnd.touch("out", (m * F + off + j) * esz, 4 * esz, ok)
                        continue
                    # mask application (mask_mlp_forward_apply): complex rows r0, r0 + 1 of row m
                    fr, ch, ns, st = apply["frames"], apply["channels"], apply["stems"], apply["stem"]
                    fbins = F // (2 * ch)
                    mm = np.minimum(m, M - 1)
                    bb, tt = mm // fr, mm % fr
                    for q in range(2):
                        r = (off + j) // 2 + q
                        f, c = r // ch, r % ch
                        bnd.touch("est", ((((bb * ns + st) * ch + c) * fbins + f) * fr + tt) * 8, 8, ok)
    return bnd


def _replay_me_fwd_reg(bnd, widths, offs, M, H, esz, vec4):
    """mask_estimator.hip me_fwd_kernel: (band, 64 GLU outputs) groups x 128-row tiles; A = 64 left and
    64 gate rows of W_b (LeftGateLoader row map), B = x rows; epilogue stores pre and out."""
    nb, F = len(widths), int(sum(widths))
    max_l = cdiv(max(widths), 64)
    mtiles = cdiv(M, 128)
    bnd.sizes["lds"] = gemm_lds_bytes(esz, 128, 128)
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    nk = cdiv(H, CHUNK_K)
    kbeg = H - nk * CHUNK_K
    # the even schedule over the existing (band, row tile, chunk) blocks; the XcdGrid past 256 bands
    units = lambda b: cdiv(widths[b], 64)
    sc = build_even_sched(nb, mtiles, units)
    if sc is not None:
        dec = sched_decode(sc, nb, units, False, bnd, "me_fwd")
        combos = sorted({(b * max_l + sub, mt) for b, mt, sub in dec if mt in (0, mtiles - 1)})
    else:
        grp, mt, valid = xcd_decode(nb * max_l, mtiles)
        combos = sorted({(int(g), int(m)) for g, m, v in zip(grp, mt, valid) if v and int(m) in (0, mtiles - 1)})
    for g_, mtile in combos:
        band, l0 = g_ // max_l, (g_ % max_l) * 64
        off, I = int(offs[band]), int(widths[band])
        if l0 >= I:
            continue
        m0 = mtile * 128
        rv = min(M - m0, 128)
        r = krow_rows(tid, 128)
        l = l0 + (r & 63)
        lc = np.minimum(l, I - 1)
        src = np.where(r < 64, lc, I + lc)
        krow_loader(bnd, "weight", esz, 2 * off * H, H, 128, H, 128, vec4, kbeg, nk, tid, row_map=(src, l < I))
        krow_loader(bnd, "x", esz, (m0 * nb + band) * H, nb * H, rv, H, 128, vec4, kbeg, nk, tid)
        for i in range(4):
            ll = l0 + i * 16 + 4 * (lane >> 4)
            okl = ll < I
            for rr in range(4):
                bnd.touch("bias", (2 * off + ll + rr) * esz, esz, okl & (ll + rr < I))
                bnd.touch("bias", (2 * off + I + ll + rr) * esz, esz, okl & (ll + rr < I))
            for j in range(2):
                m = wave * 32 + j * 16 + (lane & 15)
                ok = okl & (m < rv)
                w = 4 if vec4 else 1
                for rr in range(4 // w):
                    okr = ok & (ll + rr < I)
                    bnd.touch("pre", ((m0 + m) * 2 * F + 2 * off + ll + rr) * esz, w * esz, okr)
                    bnd.touch("pre", ((m0 + m) * 2 * F + 2 * off + I + ll + rr) * esz, w * esz, okr)
                    bnd.touch("out", ((m0 + m) * F + off + ll + rr) * esz, w * esz, okr)
    bnd.touch("offsets", np.arange(nb + 1) * 8, 8)


def _replay_me_dx_reg(bnd, widths, offs, M, H, esz, tanh_in):
    """mask_estimator.hip me_bwd_dx_kernel: (band, 128 hidden) groups x 64-row tiles, K = 2 I_b."""
    nb, F = len(widths), int(sum(widths))
    hch = cdiv(H, 128)
    mtiles = cdiv(M, 64)
    grp, mt, valid = xcd_decode(nb * hch, mtiles)
    bnd.sizes["lds"] = max(bnd.sizes["lds"], gemm_lds_bytes(esz, 128, 64))
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    v4 = True
    combos = sorted({(int(g), int(m)) for g, m, v in zip(grp, mt, valid) if v and int(m) in (0, mtiles - 1)})
    for g_, mtile in combos:
        band, h0 = g_ // hch, (g_ % hch) * 128
        off, I = int(offs[band]), int(widths[band])
        K = 2 * I
        nk = cdiv(K, CHUNK_K)
        kbeg = K - nk * CHUNK_K
        m0 = mtile * 64
        rv = min(M - m0, 64)
        mn_loader(bnd, "weight", esz, 2 * off * H + h0, H, H - h0, K, 128, v4, kbeg, nk, tid)
        krow_loader(bnd, "workspace", esz, m0 * 2 * F + 2 * off, 2 * F, rv, K, 64, v4, kbeg, nk, tid)
        hr, mc = (wave >> 1) * 64, (wave & 1) * 32
        for i in range(4):
            h = h0 + hr + i * 16 + 4 * (lane >> 4)
            for j in range(2):
                m = mc + j * 16 + (lane & 15)
                ok = (h < H) & (m < rv)
                idx = ((m0 + m) * nb + band) * H + h
                if tanh_in:
                    bnd.touch("x", idx * esz, 4 * esz, ok)
                bnd.touch("dx", idx * esz, 4 * esz, ok)


def _replay_me_dw_reg(bnd, widths, offs, M, H, esz):
    """mask_estimator.hip me_bwd_dw_kernel: (band, 128 hidden) groups x 64-wide j chunks, K = M; the
    blocks of hidden tile 0 also sum dpre over the rows (dbias)."""
    nb, F = len(widths), int(sum(widths))
    ht = cdiv(H, 128)
    maxj = cdiv(2 * max(widths), 64)
    tid = np.arange(GEMM_THREADS)
    lane, wave = tid & 63, tid >> 6
    nk = cdiv(M, CHUNK_K)
    kbeg = M - nk * CHUNK_K
    # the even schedule over the existing (band, hidden tile, j chunk) blocks (sub = hidden tile x
    # the band's j chunks + j chunk); the XcdGrid past 256 bands
    nj = lambda b: cdiv(2 * widths[b], 64)
    units = lambda b: ht * nj(b)
    sc = build_even_sched(nb, 1, units)
    if sc is not None:
        dec = sched_decode(sc, nb, units, False, bnd, "me_bwd_dw")
        pairs = sorted({(b * ht + sub // nj(b), sub % nj(b)) for b, _, sub in dec})
    else:
        grp, jc, valid = xcd_decode(nb * ht, maxj)
        pairs = sorted({(int(g), int(j)) for g, j, v in zip(grp, jc, valid) if v})
    for g_, j_ in pairs:
        band, h0 = g_ // ht, (g_ % ht) * 128
        j0 = j_ * 64
        off, I = int(offs[band]), int(widths[band])
        K2 = 2 * I
        if j0 >= K2 or M == 0:
            continue
        mn_loader(bnd, "x", esz, band * H + h0, nb * H, H - h0, M, 128, True, kbeg, nk, tid)
        mn_loader(bnd, "workspace", esz, 2 * off + j0, 2 * F, K2 - j0, M, 64, True, kbeg, nk, tid)
        if h0 == 0:
            bnd.touch("dbias", (2 * off + j0 + tid) * esz, esz, (tid < 64) & (tid < K2 - j0))
        hr, jcol = (wave >> 1) * 64, (wave & 1) * 32
        for i in range(4):
            h = h0 + hr + i * 16 + 4 * (lane >> 4)
            for j in range(2):
                jj = j0 + jcol + j * 16 + (lane & 15)
                bnd.touch("dw", (2 * off * H + jj * H + h) * esz, 4 * esz, (h < H) & (jj < K2))


# ----------------------------------------------------------------------------- row kernels


def _row_geom(dim: int, vec: int):
    """rowgeom.h pick_row_geom for aligned pointers."""
    if dim % vec == 0:
        nvec = dim // vec
        tl = 0
        while tl < 6 and nvec % (2 << tl) == 0:
            tl += 1
        nv = nvec >> tl
        if 1 <= nv <= 4:
            return vec, nv, tl
    if dim <= 512:
        need = cdiv(dim, WAVE)
        nv = 1 if need <= 1 else 2 if need <= 2 else 4 if need <= 4 else 8
        return 1, nv, 6
    return None


def replay_rms_norm(rows: int, dim: int, esz: int):
    """rmsnorm.hip rms_fwd_kernel and rms_bwd_kernel (saved input), col_sum_kernel."""
    sizes = {"x": rows * dim * esz, "gamma": dim * esz, "out": rows * dim * esz, "inv_norm": rows * 4,
             "dy": rows * dim * esz, "dx": rows * dim * esz, "dgamma": dim * esz,
             "workspace": 1024 * dim * 4, "red": 8 * dim * 4}
    bnd = Bounds(sizes)
    geo = _row_geom(dim, 16 // esz)
    if geo is None:
        bnd.fail("rms: unsupported dim")
        return bnd
    vec, nv, tl = geo
    half = False
    if vec == 16 // esz and nv == 3 and vec >= 4:
        h = _row_geom(dim, vec // 2)
        if h is not None and h[0] == vec // 2 and h[1] == 3 and h[2] == tl + 1:
            vec, nv, tl, half = h[0], h[1], h[2], True
    guard = vec == 1
    for threads, kind in ((256, "fwd"), (512, "bwd")):
        tid = np.arange(threads)
        lane, wave = tid & 63, tid >> 6
        tpr = 1 << tl
        t, slot = lane & (tpr - 1), lane >> tl
        rpw = WAVE >> tl
        rpb = rpw * (threads // WAVE)
        nblk = cdiv(rows, rpb)
        grid = min(nblk, 65536) if kind == "fwd" else min(nblk, 1024)
        for base in sorted({0, (nblk - 1) * rpb}):
            row = base + wave * rpw + slot
            valid = row < rows
            rl = np.where(valid, row, rows - 1)
            for v in range(nv):
                col = (v * tpr + t) * vec
                okc = col < dim
                ld = okc if guard else np.ones_like(okc)
                srcs = ("x",) if kind == "fwd" else ("dy", "x")
                for b in srcs:
                    bnd.touch(b, (rl * dim + col) * esz, vec * esz, ld & (valid if guard else True))
                bnd.touch("gamma", col * esz, vec * esz, okc)
                dst = "out" if kind == "fwd" else "dx"
                bnd.touch(dst, (row * dim + col) * esz, vec * esz, valid & okc)
                if kind == "bwd":
                    bnd.touch("red", (wave * dim + col) * 4, vec * 4, (slot == 0) & okc)
            if kind == "fwd":
                bnd.touch("inv_norm", row * 4, 4, valid & (t == 0))
            else:
                bnd.touch("inv_norm", rl * 4, 4)
        if kind == "bwd":
            parts = grid
            for blk in sorted({0, parts - 1}):
                c = np.arange(dim)
                bnd.touch("workspace", (blk * dim + c) * 4, 4)
            _replay_col_sum(bnd, "workspace", parts, dim, "dgamma", esz)
    _ = half
    return bnd


def replay_rotary_qkv(B: int, N: int, H: int, D: int, esz: int, backward: bool):
    """rotary.hip rotary_kernel with the three parts of a fused qkv projection (extension.py
    rotary_qkv_forward / _backward strides); tables are the [..., ::2] views of [1, N, 1, D]."""
    HD = H * D
    sizes = {"qkv": B * N * 3 * HD * esz, "o0": B * N * HD * esz, "o1": B * N * HD * esz,
             "o2": B * N * HD * esz, "cos": N * D * esz, "sin": N * D * esz}
    bnd = Bounds(sizes)
    dense_bhnd = (H * N * D, D, N * D)  # [B, H, N, D] buffer seen as [B, N, H, D]
    qkv = (N * 3 * HD, 3 * HD, D)
    if not backward:
        ins = [("qkv", p * HD, qkv) for p in range(3)]
        outs = [(f"o{p}", 0, dense_bhnd) for p in range(3)]
    else:
        ins = [(f"o{p}", 0, dense_bhnd) for p in range(3)]
        outs = [("qkv", p * HD, qkv) for p in range(3)]
    vec = 16 // esz
    while vec > 2 and any(s % vec for _, _, st in ins + outs for s in st):
        vec //= 2
    packs = B * N * H * D // vec
    # the grid-stride loop visits every pack index (packs past the end redo the last one); a pack's
    # addresses depend on its index only and grow with (b, n, h, d), so the first and the last
    # 64K packs hold every extreme
    span = min(packs, 1 << 16)
    i = np.unique(np.concatenate([np.arange(span), np.arange(packs - span, packs)])).astype(np.int64)
    ppt = HD // vec
    tok = i // ppt
    e = (i - tok * ppt) * vec
    b, n = tok // N, tok % N
    h, d = e // D, e % D
    cs_seq = D
    for part in range(3):
        ib, ioff, si = ins[part]
        ob, ooff, so = outs[part]
        bnd.touch(ib, (ioff + b * si[0] + n * si[1] + h * si[2] + d) * esz, vec * esz)
        if part < 2:
            for tb in ("cos", "sin"):
                # repeated-table mode: 16 bytes from element 2 * (d / 2) of the position's row
                bnd.touch(tb, (n * cs_seq + 2 * (d >> 1)) * esz, vec * esz)
        bnd.touch(ob, (ooff + b * so[0] + n * so[1] + h * so[2] + d) * esz, vec * esz)
    return bnd


def replay_attention_gate(B: int, N: int, H: int, Dh: int, dim: int, esz: int):
    """attn_gate.hip gate_fwd_kernel / gate_bwd_kernel (fast path) with attn and grad_attn the
    [B, N, H, Dh] views of dense [B, H, N, Dh] SDPA buffers, col_sum of the partials."""
    rows = B * N
    HD = H * Dh
    sizes = {"attn": B * N * HD * esz, "x": rows * dim * esz, "weight": H * dim * esz, "bias": H * esz,
             "out": rows * HD * esz, "gate": rows * H * esz, "grad_out": rows * HD * esz,
             "grad_attn": B * N * HD * esz, "grad_x": rows * dim * esz, "grad_weight": H * dim * esz,
             "grad_bias": H * esz, "lds": (2 * H * dim + H) * 4}
    chunks_per = 64
    while cdiv(rows, chunks_per) > 2048:
        chunks_per *= 2
    parts_ws = max(cdiv(rows, chunks_per), 1024)
    ws_gpre = cdiv(rows * H * 4, 256) * 256
    ws_pw = cdiv(parts_ws * H * dim * 4, 256) * 256
    sizes["workspace"] = ws_gpre + ws_pw + cdiv(parts_ws * H * 4, 256) * 256
    bnd = Bounds(sizes)
    E = HD // WAVE
    logh = H.bit_length() - 1
    jx = cdiv(dim, WAVE)
    jx = jx if jx <= 4 else 8
    fast = (1 << logh) == H and 1 <= logh <= 4 and HD % WAVE == 0 and E in (2, 4, 8) and cdiv(dim, WAVE) <= 8 \
        and H * jx <= 64 and (2 * H * dim + H) * 4 <= 48 * 1024
    if not fast:
        bnd.fail("gate: generic path not modelled")
        return bnd
    sb, sn, sh = HD * N, Dh, N * Dh  # transposed view of [B, H, N, Dh]
    LPH = WAVE // H
    tid = np.arange(256)
    lane, wave = tid & 63, tid >> 6
    head, sub = lane // LPH, lane % LPH
    k = np.arange(H * dim)
    bnd.touch("weight", k * esz, esz)
    bnd.touch("lds", ((k % dim) * H + k // dim) * 4, 4)
    # the grids: up to 4096 / 1024 blocks, fewer where fewer fit on the device at once (any count works:
    # the loops stride over the grid); both ends are replayed
    for kind, maxb in (("fwd", 4096), ("fwd", 1792), ("bwd", 1024), ("bwd", 768)):
        nblk = min(cdiv(rows, 4 * 2), maxb)
        for blk in sorted({0, nblk - 1}):
            # a wave's rows: m0 = (block * 4 + wave) * 2 + trip * (grid * 8) while m0 < rows; the
            # loads of a live trip read rows clamped to the last one, the stores only rows < rows
            first = (blk * 4 + wave) * 2
            trips = np.where(first < rows, (rows - 1 - first) // (nblk * 8), -1)
            for m0, live in ((first, first < rows), (first + np.maximum(trips, 0) * nblk * 8, trips >= 0)):
                for r in range(2):
                    m = m0 + r
                    ok = live & (m < rows)
                    mc = np.minimum(m, rows - 1)
                    bb, nn = mc // N, mc % N
                    tokc = bb * sb + nn * sn + head * sh + sub * E
                    bnd.touch("attn", tokc * esz, E * esz, live)
                    for j in range(jx):
                        i = lane + j * WAVE
                        bnd.touch("x", (mc * dim + np.where(i < dim, i, 0)) * esz, esz, live)
                        if kind == "bwd":
                            bnd.touch("grad_x", (m * dim + i) * esz, esz, ok & (i < dim))
                            bnd.touch("lds", (i * H + head) * 4, 4, ok & (i < dim))
                    if kind == "fwd":
                        bnd.touch("gate", (m * H + head) * esz, esz, ok & (sub == 0))
                        bnd.touch("out", (m * HD + lane * E) * esz, E * esz, ok)
                    else:
                        bnd.touch("grad_out", (mc * HD + lane * E) * esz, E * esz, live)
                        bnd.touch("gate", (mc * H + head) * esz, esz, live)
                        bnd.touch("grad_attn", tokc * esz, E * esz, ok)
        if kind == "bwd":
            for j in range(jx):
                i = lane + j * WAVE
                for h in range(H):
                    bnd.touch("lds", (H * dim + h * dim + i) * 4, 4, i < dim)
            bnd.touch("lds", (H * dim + H * dim + head) * 4, 4, sub == 0)
            c = np.arange(H * dim)
            for blk in sorted({0, nblk - 1}):
                bnd.touch("workspace", ws_gpre + (blk * H * dim + c) * 4, 4)
                bnd.touch("workspace", ws_gpre + ws_pw + (blk * H + np.arange(H)) * 4, 4)
            _replay_col_sum(bnd, "workspace", nblk, H * dim, "grad_weight", esz, poff=ws_gpre)
            _replay_col_sum(bnd, "workspace", nblk, H, "grad_bias", esz, poff=ws_gpre + ws_pw)
    bnd.touch("bias", head * esz, esz)
    return bnd


# ----------------------------------------------------------------------------- configs


BSR_WIDTHS = tuple([8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516])

# (name, band widths, rows M = B * T, model dim, mask hidden, q/k shapes (B*NB, T) and (B*T, NB))
CONFIG_SHAPES = {
    "configs0": (BSR_WIDTHS, 130, 64, 256, (124, 65, 4, 32), (130, 62, 4, 32)),
    "configs1": (BSR_WIDTHS, 1032, 192, 768, (248, 258, 8, 64), (1032, 62, 8, 64)),
    "configs4": (BSR_WIDTHS, 1896, 512, 2048, (124, 948, 8, 64), (1896, 62, 8, 64)),
}


def mel_widths():
    """The 60-band Mel layout (4 * bins per band) of configs[3], from the restated model."""
    from pymsst_amd.core.mel_band_roformer import mel_band_bins

    return tuple(4 * len(b) for b in mel_band_bins(44100, 2048, 60))


def all_replays(name: str, esz: int):
    """Every kernel replay of one configuration's fused train step (band split fwd/bwd, grouped
    linear fwd/bwd of the mask hidden layer, mask final fwd/bwd, RMSNorm at the model dim, fused qkv
    rotary and the attention output gate on both attention axes); yields (label, Bounds)."""
    if name == "configs3":
        widths, M, dim, hidden = mel_widths(), 2760, 192, 768
        qk = [(240, 690, 8, 64), (2760, 60, 8, 64)]
    else:
        widths, M, dim, hidden, qk_t, qk_f = CONFIG_SHAPES[name]
        qk = [qk_t, qk_f]
    nb = len(widths)
    yield "band_split_fwd", replay_band_split_forward(widths, M, dim, esz)
    yield "band_split_bwd", replay_band_split_backward(widths, M, dim, esz)
    if esz == 2 and name != "configs0":  # autocast configs: the band split of the fp32 STFT input
        yield from replay_band_split_mixed(widths, M, dim)
    yield "grouped_linear_fwd", replay_band_split_forward([dim] * nb, M, hidden, esz, norm=False, act_tanh=True)
    yield "grouped_linear_bwd", replay_band_split_backward([dim] * nb, M, hidden, esz, grouped=True)
    yield "mask_final_fwd", replay_mask_final_forward(widths, M, hidden, esz)
    yield "mask_final_bwd", replay_mask_final_backward(widths, M, hidden, esz, tanh_in=True)
    if esz == 2:
        yield "mask_mlp_fwd", replay_mask_mlp_forward(widths, M, dim, hidden, esz)
        if name in ("configs1", "configs4"):  # BS-RoFormer: stereo, bins x 2 channels x (re, im)
            frames = {"configs1": 258, "configs4": 948}[name]
            stems = {"configs1": 4, "configs4": 1}[name]
            yield "mask_mlp_fwd_apply", replay_mask_mlp_forward(
                widths, M, dim, hidden, esz, apply={"frames": frames, "channels": 2, "stems": stems, "stem": stems - 1})
    yield "rms_norm", replay_rms_norm(M * nb, dim, esz)
    for shape in qk:
        yield f"attention_gate{list(shape)}", replay_attention_gate(shape[0], shape[1], shape[2], shape[3], dim, esz)
        for bwd in (False, True):
            yield f"rotary_qkv{'_bwd' if bwd else ''}{list(shape)}", replay_rotary_qkv(*shape, esz, bwd)
