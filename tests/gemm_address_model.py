"""Host-side address model of the grouped-GEMM kernels (bebelm_amd/csrc/bb_prefill.hip).

Test infrastructure, not product code: it restates, in Python, the index arithmetic by which
k_gemm, k_gemm_wide and k_gateup16 choose their tiles, member rows, copy sources and output
rows, so that every address a launch can touch is checked against the size of the buffer it
belongs to on the CPU, for any routing, before a shape ever runs on the GPU.

What is modelled (per block of the launch the host code in launch_gemm would make):
  * the launch choice (k_gateup16 / k_gemm with member tiles of 16, 64, 80 or 128 / k_gemm_wide)
    and its grid;
  * the block -> (member tile, row tile) mapping, including the XCD-aware order;
  * the member tile: expert, first member, count, group base (find_tile, expert_tile,
    hit_expert_tile, find_wide_tile), and the member rows and output rows (member_rows,
    member_rows_list, the all-tokens form);
  * every copy stream over all super-blocks: weight tile-blocks, activation chunks, the Q4_K
    min-term records (when the launch reads them), scales (raw
    global addresses for the plain forms, buffer-resource ranges for the buffer forms: a buffer
    access past its range reads zero, so for those the range itself must lie inside the buffer);
  * every output store.
Buffers are sized as the library allocates them: the packed experts E * stride, the x / act
quantisation T * n_in (or n_ent * n_in) bytes and their scales, the outputs n_ent rows.
A check also confirms that the stores of real members cover every output row exactly once.
"""
from dataclasses import dataclass

import numpy as np

QK = 256
Q4_K, Q6_K = 12, 14
TB = {Q4_K: 9216, Q6_K: 13440}  # bytes of one packed tile-block (64 rows x one super-block)
GATEUP, DOWN = 0, 1
WIDE_LOG, WIDE_NB, WIDE_MIN_AVG = 4, 256, 192
GU16_WAVES = 16
GEMM_MS_MIN_AVG = 128
MAX_ENTRIES = 64 * 8  # SEL_REGS * 512 of the in-block member lists (bb_members.h)


def route_bufs(sel, E):
    """counts, offsets, perm of the stable grouping (model.rs:316-322) and per-expert lists."""
    sel = np.asarray(sel, np.int64).reshape(-1)
    counts = np.bincount(sel, minlength=E)[:E]
    offsets = np.concatenate([[0], np.cumsum(counts)])
    perm = np.argsort(sel, kind="stable")
    lists = [np.nonzero(sel == e)[0] for e in range(E)]
    return counts, offsets, perm, lists


@dataclass
class Shape:
    dt: int
    kind: int
    T: int
    n_in: int
    n_out: int
    E: int
    K: int
    quant: bool = True  # the MoE block's gate/up launch gets the act rows' Q8 buffers

    @property
    def n_ent(self):
        return self.T * self.K

    @property
    def nb(self):
        return self.n_in // QK

    @property
    def n_t64(self):
        return self.n_out // 32 if self.kind == GATEUP else self.n_out // 64

    @property
    def tile_bytes(self):
        return self.nb * TB[self.dt]

    @property
    def stride(self):
        return self.n_t64 * self.tile_bytes

    @property
    def x_rows(self):
        return self.T if self.kind == GATEUP else self.n_ent


class Violations(list):
    def add(self, what):
        if len(self) < 50:
            self.append(what)


def reads_ms(s):
    """gemm_reads_ms: the caller carves the min-term records and the Q4_K GEMM reads them."""
    return s.dt == Q4_K and s.n_ent >= GEMM_MS_MIN_AVG * s.E


def launch_choice(s):
    """launch_gemm's choice: ('wide', n_mt) / ('gateup16', n_blocks) / ('gemm', mt, n_mt, buf)."""
    n_ent, E = s.n_ent, s.E
    if s.dt == Q6_K and s.kind == DOWN and n_ent >= WIDE_MIN_AVG * E and n_ent * s.n_in < (1 << 31):
        return ("wide", (n_ent // WIDE_NB + (WIDE_LOG + 1) * E + 7) // 8 * 8)
    mt = 8 if s.dt == Q6_K and n_ent >= 128 * E else (4 if n_ent >= 16 * E else 1)
    if s.dt == Q4_K and mt == 4 and n_ent >= 48 * E and not reads_ms(s):
        mt = 5 if E > 1 or (n_ent + 79) // 80 * 5 < (n_ent + 63) // 64 * 4 else 4
    if (s.dt == Q4_K and s.kind == GATEUP and mt == 1 and s.quant and s.T <= 16 and n_ent <= 64 and E <= 32
            and s.n_out % QK == 0 and s.n_in in (2048, 512)):
        return ("gateup16", E * (s.n_out // QK))  # blocks of 16 waves over 256 outputs of one expert
    bn = 16 * mt
    n_mt = E * ((s.T + bn - 1) // bn) if mt == 1 else ((n_ent + bn - 1) // bn + E + 7) // 8 * 8
    buf = s.x_rows * s.n_in < (1 << 31) and 2 * s.tile_bytes < (1 << 31)
    return ("gemm", mt, n_mt, buf)


def _check_range(v, what, lo, hi, size):
    if lo < 0 or hi > size:
        v.add(f"{what}: [{lo}, {hi}) outside [0, {size})")


def _block_order(lin, n_mt, n_rt, mt):
    if mt == 1:
        return lin // n_rt, lin % n_rt
    xcd, slot = lin & 7, lin >> 3
    mt_local, rt_step = slot // n_rt, slot % n_rt
    return mt_local * 8 + xcd, (n_rt - 1 - rt_step) if (mt_local & 1) else rt_step


def check_gemm(s, sel, v, written):
    _, mt, n_mt, buf = launch_choice(s)
    counts, offsets, perm, lists = route_bufs(sel, s.E)
    E, K, bn, nb, tbytes = s.E, s.K, 16 * mt, s.nb, s.tile_bytes
    n_rt = s.n_t64 // 2
    w_size, xq_size, sx_size = E * s.stride, s.x_rows * s.n_in, s.x_rows * nb * 4
    ms = mt == 4 and buf and reads_ms(s)  # the f16 min-term form (k_gemm<.., 4, true, true>)
    ms_size = s.x_rows * nb * 32  # 16 halves per row and super-block
    out_size = s.n_ent * s.n_out * 4
    if mt == 1 and s.n_ent > MAX_ENTRIES:
        v.add(f"member lists hold {MAX_ENTRIES} entries, the call has {s.n_ent}")
        return
    hit = [e for e in range(E) if counts[e] > 0]
    # all tiles of the grouping (the MT > 1 enumeration of find_tile)
    tiles = [(e, t * bn) for e in range(E) for t in range((counts[e] + bn - 1) // bn)]
    for lin in range(n_mt * n_rt):
        mtile, rtile = _block_order(lin, n_mt, n_rt, mt)
        if mtile >= n_mt:
            v.add(f"block {lin}: member tile {mtile} beyond the grid's {n_mt}")
            continue
        if 2 * rtile + 2 > s.n_t64:
            v.add(f"block {lin}: row tile {rtile} beyond the expert's {s.n_t64} packed tiles")
            continue
        all_tokens = mt == 1 and s.kind == GATEUP and s.T <= 16
        if mt == 1:
            e0, mt_e = mtile % E, mtile // E
            if s.kind == DOWN and mt_e == 0:  # weights requested before the selections are read
                _check_range(v, f"block {lin}: early weights", e0 * s.stride + 2 * rtile * tbytes,
                             e0 * s.stride + 2 * rtile * tbytes + 2 * tbytes, w_size)
            if s.kind == GATEUP:
                if e0 >= len(hit):
                    continue
                e = hit[e0]
            else:
                e = e0
            if mt_e * bn >= counts[e]:
                continue
            m0, g = mt_e * bn, counts[e]
            cnt, base = min(bn, g - m0), int(offsets[e])
            lst = lists[e]
            if all_tokens:
                rows = [min(n, s.T - 1) for n in range(bn)]
                outs = [-1] * bn
                for j in range(cnt):
                    outs[lst[j] // K] = base + j
            else:
                rows, outs = [], []
                for n in range(bn):
                    j = m0 + min(n, cnt - 1)
                    ent = int(lst[j])
                    rows.append(ent // K if s.kind == GATEUP else base + j)
                    outs.append((base + j if s.kind == GATEUP else ent) if n < cnt else -1)
        else:
            if mtile >= len(tiles):
                continue
            e, m0 = tiles[mtile]
            g, base = counts[e], int(offsets[e])
            cnt = min(bn, g - m0)
            rows, outs = [], []
            for n in range(bn):
                pos = base + m0 + min(n, cnt - 1)
                if not 0 <= pos < s.n_ent:
                    v.add(f"block {lin}: group position {pos} outside [0, {s.n_ent})")
                    pos = 0
                ent = int(perm[pos])
                rows.append(ent // K if s.kind == GATEUP else pos)
                outs.append((pos if s.kind == GATEUP else ent) if n < cnt else -1)
        w0 = e * s.stride + 2 * rtile * tbytes
        # weight copies of every super-block: tile-blocks of the block's two packed tiles
        _check_range(v, f"block {lin}: weights", w0, w0 + tbytes + (nb - 1) * TB[s.dt] + TB[s.dt], w_size)
        for m, r in enumerate(rows):
            if not 0 <= r < s.x_rows:
                v.add(f"block {lin}: member {m} reads row {r} of {s.x_rows}")
                continue
            _check_range(v, f"block {lin}: activations of member {m}", r * s.n_in, r * s.n_in + s.n_in, xq_size)
            _check_range(v, f"block {lin}: scales of member {m}", 4 * r * nb, 4 * (r * nb + nb), sx_size)
            if ms:
                _check_range(v, f"block {lin}: min-term records of member {m}", 32 * r * nb, 32 * (r * nb + nb),
                             ms_size)
        if buf:  # the buffer resources' ranges themselves
            _check_range(v, f"block {lin}: weight resource", w0, w0 + 2 * tbytes, w_size)
        if ms:
            _check_range(v, f"block {lin}: min-term resource", 0, s.x_rows * nb * 32, ms_size)
        # output stores: 2 packed tiles x 64 rows -> columns of this row tile
        for k64 in range(2):
            t64 = 2 * rtile + k64
            cols = range(32 * t64, 32 * t64 + 32) if s.kind == GATEUP else range(64 * t64, 64 * t64 + 64)
            for o in outs:
                if o < 0:
                    continue
                for col in (cols[0], cols[-1]):
                    _check_range(v, f"block {lin}: store", 4 * (o * s.n_out + col), 4 * (o * s.n_out + col) + 4,
                                 out_size)
                written[o, cols.start:cols.stop] += 1


def check_wide(s, sel, v, written):
    _, n_mt = launch_choice(s)
    counts, offsets, perm, _ = route_bufs(sel, s.E)
    E, K, nb, tbytes = s.E, s.K, s.nb, s.tile_bytes
    n_rt = s.n_t64 // 2
    w_size, out_size = E * s.stride, s.n_ent * s.n_out * 4
    if s.x_rows * s.n_in >= (1 << 32) or s.x_rows * nb * 4 >= (1 << 32):
        v.add("activation resources exceed 32-bit ranges")
    # chunk enumeration of find_wide_tile: class k = chunks of 16 >> k member tiles
    chunks = []
    for k in range(WIDE_LOG + 1):
        for e in range(E):
            st = (counts[e] + 15) >> 4
            n_k = st >> WIDE_LOG if k == 0 else (st >> (WIDE_LOG - k)) & 1
            m0 = sum(((st >> WIDE_LOG) if kk == 0 else (st >> (WIDE_LOG - kk)) & 1) * (WIDE_NB >> kk) for kk in range(k))
            for i in range(n_k):
                chunks.append((e, m0 + i * (WIDE_NB >> k), (1 << WIDE_LOG) >> k))
    for lin in range(n_mt * n_rt):
        mtile, rtile = _block_order(lin, n_mt, n_rt, 2)
        if mtile >= len(chunks):
            continue
        e, m0, nt = chunks[mtile]
        g, base = counts[e], int(offsets[e])
        cnt = min(16 * nt, g - m0)
        if cnt <= 0:
            v.add(f"wide block {lin}: chunk with no members")
            continue
        for wave4 in range(2):
            t64 = 2 * rtile + wave4
            if t64 >= s.n_t64:
                v.add(f"wide block {lin}: packed tile {t64} of {s.n_t64}")
                continue
            wt = e * s.stride + t64 * tbytes
            _check_range(v, f"wide block {lin}: weight resource", wt, wt + tbytes, w_size)
            cols = range(32 * t64, 32 * t64 + 32) if s.kind == GATEUP else range(64 * t64, 64 * t64 + 64)
            for n in range(16 * nt):
                pos = base + m0 + min(n, cnt - 1)
                if not 0 <= pos < s.n_ent:
                    v.add(f"wide block {lin}: group position {pos}")
                    continue
                ent = int(perm[pos])
                row = ent // K if s.kind == GATEUP else pos
                if not 0 <= row < s.x_rows:
                    v.add(f"wide block {lin}: row {row} of {s.x_rows}")
                if n < cnt:
                    o = pos if s.kind == GATEUP else ent
                    _check_range(v, f"wide block {lin}: store", 4 * (o * s.n_out + cols[0]),
                                 4 * (o * s.n_out + cols[-1]) + 4, out_size)
                    written[o, cols.start:cols.stop] += 1


def check_gateup16(s, sel, v, written):
    _, n_blocks = launch_choice(s)
    counts, offsets, _, lists = route_bufs(sel, s.E)
    E, K, NB, tbytes = s.E, s.K, s.nb, s.tile_bytes
    n_ot = s.n_out // 16
    w_size, out_size = E * s.stride, s.n_ent * s.n_out * 4
    sel_alloc = (s.n_ent * 4 + 255) // 256 * 256  # the workspace carve rounds to 256 bytes
    if 64 * 4 > sel_alloc:
        v.add(f"gateup16 reads 64 selections from a carve of {sel_alloc} bytes")
    if s.n_ent > 64:
        v.add("gateup16 with more than 64 entries")
    NW = GU16_WAVES
    aq_size, aqs_size = s.n_ent * s.n_out, s.n_ent * (s.n_out // QK) * 4
    qwritten = np.zeros((s.n_ent, s.n_out // QK), np.int32)
    for b in range(n_blocks):
        if (b * NW) // n_ot != (b * NW + NW - 1) // n_ot:
            v.add(f"gateup16 block {b} spans two experts")
        for w in range(NW):
            # activation and scale copies: rows clamped to the batch, super-blocks below NB
            for t in range((4 * NB + NW - 1) // NW):
                j = min(w + NW * t, 4 * NB - 1)
                bb, mm = j >> 2, 4 * (j & 3) + 3
                row = min(mm, s.T - 1)
                _check_range(v, "gateup16 activation copy", row * NB * QK + bb * QK, row * NB * QK + bb * QK + QK,
                             s.T * s.n_in)
            u = min(64 * w + 63, 16 * NB - 1)
            _check_range(v, "gateup16 scale copy", 4 * (min(u & 15, s.T - 1) * NB + (u >> 4)),
                         4 * (min(u & 15, s.T - 1) * NB + (u >> 4)) + 4, s.T * NB * 4)
            unit = b * NW + w
            if unit >= E * n_ot:
                continue  # its resource has range 0: every load reads zero
            e, o = unit // n_ot, unit % n_ot
            t64, t16 = o >> 1, o & 1
            wt = e * s.stride + t64 * tbytes
            _check_range(v, "gateup16 weight resource", wt, wt + tbytes, w_size)
            if counts[e] == 0:
                continue
            base = int(offsets[e])
            lst = list(lists[e])
            col0 = 32 * t64 + 16 * t16
            for n in range(min(16, s.T)):
                mine = [i for i in range(K) if n * K + i in lst]
                if not mine:
                    continue
                orow = base + lst.index(n * K + mine[0])
                _check_range(v, "gateup16 store", 4 * (orow * s.n_out + col0), 4 * (orow * s.n_out + col0 + 16),
                             out_size)
                written[orow, col0:col0 + 16] += 1
            # wave w quantises token w's 256 values at super-block col0 / 256
            if w < s.T:
                mine = [i for i in range(K) if w * K + i in lst]
                if mine:
                    orow, jb = base + lst.index(w * K + mine[0]), col0 // QK
                    _check_range(v, "gateup16 act Q8 store", orow * s.n_out + jb * QK, orow * s.n_out + jb * QK + QK,
                                 aq_size)
                    _check_range(v, "gateup16 act scale store", 4 * (orow * (s.n_out // QK) + jb),
                                 4 * (orow * (s.n_out // QK) + jb) + 4, aqs_size)
                    qwritten[orow, jb] += 1
    if not np.all(qwritten == 1):
        v.add(f"gateup16 act Q8: {(qwritten != 1).sum()} (row, super-block) pairs not written exactly once")


def check(s, sel):
    """Violations of one launch of shape s on the selections sel [T, K] (empty when in bounds),
    including outputs of real members left unwritten or written twice."""
    v = Violations()
    sel = np.asarray(sel).reshape(s.T, s.K)
    written = np.zeros((s.n_ent, s.n_out), np.int32)
    choice = launch_choice(s)[0]
    {"gemm": check_gemm, "wide": check_wide, "gateup16": check_gateup16}[choice](s, sel, v, written)
    if not v:
        if s.kind == GATEUP:
            # rows of group positions: every position's gate/up outputs (n_out = F) exactly once
            bad = np.count_nonzero(written != 1)
        else:
            bad = np.count_nonzero(written != 1)
        if bad:
            v.add(f"{bad} outputs written {sorted(set(written.reshape(-1).tolist()))} times")
    return choice, list(v)
