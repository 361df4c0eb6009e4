"""Host-side index model of the LDS use of the 16 < n <= 64 MFMA kernels (csrc/mfma32.hip), on the CPU.

Two pipelined variants of the n = 32, C = 4096 forward were withdrawn after some GPU runs returned one
wrong MFMA result element, in waves 4-7 of the workgroup only (the second wave of each SIMD).  The
shipped kernels share their slab staging, LDS layout and wave mapping, so this model restates, for
every launch shape the host code can choose, each LDS access those kernels make (array, byte range,
wave, lane, read or write) together with the synchronisation around it, and checks:

- every access stays inside its array (the dynamic arrays at the size the host launches with);
- the per-wave arrays (the staged slabs, the loop forward's y) are private: no byte is touched by two
  waves, in particular by waves w and w + 4 of one SIMD;
- every byte of a shared array that one wave writes and another wave reads or writes is separated by a
  workgroup barrier (no cross-wave access pair inside one barrier epoch);
- inside one wave, a lane that reads a byte another lane wrote does so after that write in program order
  (one wave's LDS accesses complete in order; the kernels also wait for lgkmcnt(0) there).

The constants are read from the source file, so the model follows the kernels' layout.  The index
formulas restate the kernels' expressions, each with the line range of mfma32.hip it follows.  The
withdrawn second variant (x staged through the wave's LDS slab "as the pipelined backward does") is
modelled with the pipelined backward's x staging inside the four-slab forward; the first variant staged
nothing in LDS.
"""

import re
from pathlib import Path

import numpy as np
import pytest

SRC = Path(__file__).resolve().parents[1] / "mhc-mlx_amd" / "csrc" / "mfma32.hip"


def _constants():
    """constexpr int kMf32* values of mfma32.hip, evaluated in order (they refer to each other)."""
    env = {}
    for name, expr in re.findall(r"constexpr int (kMf32\w+|kMf64\w+) = ([^;]+);", SRC.read_text()):
        env[name] = int(eval(expr, {"__builtins__": {}}, dict(env)))  # arithmetic on earlier constants only
    return env


K = _constants()
ROW = K["kMf32Row"]          # halfwords per staged row
SLAB = K["kMf32Slab"]        # halfwords per wave: x rows then g rows
PAR = K["kMf32Par"]          # floats per wave in the final parameter-sum reduction
MAXW = K["kMf32MaxWaves"]


class Trace:
    """LDS accesses of one workgroup: one entry per lane and instruction, in each wave's program order,
    tagged with the workgroup barrier epoch (the number of barriers all waves have passed)."""

    def __init__(self, waves, sizes):
        self.waves, self.sizes = waves, sizes  # sizes: array -> bytes
        self.rows = []                         # (array, lo, hi, wave, lane, is_write, epoch, instr)
        self.epoch = 0
        self.ninstr = 0

    def instr(self, array, wave, kind, lanes):
        """One LDS instruction of `wave`: lanes = [(lane, byte offset, bytes), ...]."""
        for lane, lo, nb in lanes:
            self.rows.append((array, lo, lo + nb, wave, lane, kind == "W", self.epoch, self.ninstr))
        self.ninstr += 1

    def barrier(self):
        self.epoch += 1


def check(tr, private=()):
    """The four properties of the module docstring, over 4-byte words (every access is a whole number of
    aligned words)."""
    assert tr.rows, "empty trace"
    names = sorted({r[0] for r in tr.rows})
    for name in names:
        rows = [r for r in tr.rows if r[0] == name]
        lo = np.array([r[1] for r in rows], np.int64)
        hi = np.array([r[2] for r in rows], np.int64)
        assert (lo % 4 == 0).all() and (hi % 4 == 0).all()
        assert lo.min() >= 0 and hi.max() <= tr.sizes[name], ("out of bounds", name, int(lo.min()), int(hi.max()),
                                                              tr.sizes[name])
        nw = (hi - lo) // 4
        idx = np.repeat(np.arange(len(rows)), nw)
        word = np.repeat(lo // 4, nw) + (np.arange(nw.sum()) - np.repeat(np.cumsum(nw) - nw, nw))
        wave = np.array([r[3] for r in rows], np.int64)[idx]
        lane = np.array([r[4] for r in rows], np.int64)[idx]
        wr = np.array([r[5] for r in rows], bool)[idx]
        ep = np.array([r[6] for r in rows], np.int64)[idx]
        ins = np.array([r[7] for r in rows], np.int64)[idx]
        if name in private:
            pairs = np.unique(np.stack([word, wave]), axis=1)
            _, cnt = np.unique(pairs[0], return_counts=True)
            assert cnt.max() == 1, ("per-wave array shared", name, int(pairs[0][np.argmax(cnt)]))
        else:
            # cross-wave: within one (word, epoch) with a write, one wave only
            key = word * (ep.max() + 1) + ep
            trip = np.unique(np.stack([key, wave]), axis=1)
            kk, nwaves = np.unique(trip[0], return_counts=True)
            bad = np.intersect1d(kk[nwaves > 1], np.unique(key[wr]))
            assert bad.size == 0, ("cross-wave access without a barrier between", name,
                                   int(bad[0] // (ep.max() + 1)))
        # inside a wave: no two lanes of one store instruction write the same word
        st = np.unique(np.stack([ins[wr], word[wr], lane[wr]]), axis=1)
        if st.size:
            _, cnt = np.unique(st[0] * (word.max() + 1) + st[1], return_counts=True)
            assert cnt.max() == 1, ("two lanes of one store on one word", name)
    return True


# ---------------------------------------------------------------------------------------------------
# kernels
# ---------------------------------------------------------------------------------------------------

LANES = [(lane, lane >> 4, lane & 15) for lane in range(64)]  # lane, q, r


def _stage_slab(tr, wave, parts=(0, 32 * ROW)):
    """x and g of a slab into the wave's rows: u32x4 stores at [(8q + e) * ROW + 8r] of xs and of
    gs = xs + 32 ROW (mf32_bwd_kernel mfma32.hip:874-881; mf32_bwd_wide_kernel and mf32_bwd_pipe_kernel
    the same expressions)."""
    base = wave * SLAB
    for part in parts:
        for e in range(8):
            tr.instr("slab", wave, "W", [(ln, 2 * (base + part + (8 * q + e) * ROW + 8 * r), 16) for ln, q, r in LANES])


def _read_dm_operands(tr, wave):
    """dM operands: u32x4 loads at [(16I + r) ROW + 32kk + 8q] of gs and of xs (mfma32.hip:901-908)."""
    base = wave * SLAB
    for kk in range(4):
        for I in range(2):
            for part in (32 * ROW, 0):
                tr.instr("slab", wave, "R",
                         [(ln, 2 * (base + part + (16 * I + r) * ROW + 32 * kk + 8 * q), 16) for ln, q, r in LANES])


def _read_own_rows(tr, wave, part):
    """The lane's own rows back: u32x4 loads at [(8q + e) ROW + 8r] (mfma32.hip:944-948, 986-990)."""
    base = wave * SLAB
    for e in range(8):
        tr.instr("slab", wave, "R", [(ln, 2 * (base + part + (8 * q + e) * ROW + 8 * r), 16) for ln, q, r in LANES])


def _rms_sums(tr, waves, it, pairs, slots):
    """s_red[2][pairs][slots] floats: lane 0 of each wave writes slot [it & 1][p][wave], a barrier, then
    every lane reads every wave's slot (backward mfma32.hip:911-926 with [2][2][kMf32MaxWaves]; forwards
    :301-308 with [2][16])."""
    for w in range(waves):
        for p in range(pairs):
            tr.instr("s_red", w, "W", [(0, 4 * (((it & 1) * pairs + p) * slots + w), 4)])
    tr.barrier()
    for w in range(waves):
        for src in range(waves):
            for p in range(pairs):
                tr.instr("s_red", w, "R", [(ln, 4 * (((it & 1) * pairs + p) * slots + src), 4) for ln, _, _ in LANES])


def _param_sums(tr, waves):
    """mf32_bwd_param_sums (mfma32.hip:758-800): after a barrier each wave writes its kMf32Par floats at
    wave kMf32Par of the reused slab memory, a barrier, then every thread reads every wave's."""
    tr.barrier()
    for w in range(waves):
        for I in range(2):
            for J in range(2):
                for k in range(4):
                    tr.instr("slab", w, "W", [(ln, 4 * (w * PAR + (16 * I + 4 * q + k) * 32 + 16 * J + r), 4)
                                              for ln, q, r in LANES])
        for e in range(8):
            tr.instr("slab", w, "W", [(ln, 4 * (w * PAR + 1024 + 8 * q + e), 4) for ln, q, r in LANES if r == 0])
            tr.instr("slab", w, "W", [(ln, 4 * (w * PAR + 1024 + 32 + 8 * q + e), 4) for ln, q, r in LANES if r == 0])
    tr.barrier()
    nthreads = waves * 64
    for w in range(waves):
        for k0 in range(0, 32 * 32 + 64, nthreads):
            for src in range(waves):
                lanes = [(ln, 4 * (src * PAR + k0 + w * 64 + ln), 4) for ln in range(64)
                         if k0 + w * 64 + ln < 32 * 32 + 64]
                if lanes:
                    tr.instr("slab", w, "R", lanes)


def _params_by_wave0(tr, name, nbytes, waves):
    """Parameters written by wave 0, a barrier, then read by every wave (s_par mfma32.hip:820-822; the
    loop forward's s_aa / s_am :423-435)."""
    tr.instr(name, 0, "W", [(ln, (ln * nbytes // 64) // 4 * 4, 4) for ln in range(64)])
    tr.barrier()
    for w in range(waves):
        tr.instr(name, w, "R", [(ln, 0, nbytes) for ln in range(64)])


def bwd_trace(waves, spw, tokens, pipe):
    """mf32_bwd_kernel (spw = 1), mf32_bwd_wide_kernel and mf32_bwd_pipe_kernel (spw > 1), one token after
    another in one workgroup; dynamic LDS max(waves kMf32Slab halfwords, waves kMf32Par floats)
    (mfma32.hip:2023-2024).  Before the RMS barrier every slab step stages x and g and reads the dM
    operands; after it (slabs last first) mf32_bwd_kernel reads g and x back from its one staged slab,
    the pipelined kernel does the same for slab SPW - 1 and stages the others again, and the wide kernel
    reads the rows from global memory (no LDS)."""
    size = max(waves * SLAB * 2, waves * PAR * 4)
    tr = Trace(waves, {"slab": size, "s_red": 2 * 2 * MAXW * 4, "s_par": 4096})
    _params_by_wave0(tr, "s_par", 4096, waves)
    # every slab step touches the same rows of the wave's buffer, so three steps stand for any SPW (the
    # pipelined kernel's first post-barrier step, the one that reads the slab staged last, is kept)
    spw = min(spw, 3)
    for it in range(tokens):
        for w in range(waves):
            for _ in range(spw):
                _stage_slab(tr, w)
                _read_dm_operands(tr, w)
        _rms_sums(tr, waves, it, 2, MAXW)
        for w in range(waves):
            for s in reversed(range(spw)):
                if spw == 1 or (pipe and s == spw - 1):
                    _read_own_rows(tr, w, 32 * ROW)
                    _read_own_rows(tr, w, 0)
                elif pipe:
                    _stage_slab(tr, w)
                    _read_own_rows(tr, w, 32 * ROW)
                    _read_own_rows(tr, w, 0)
    _param_sums(tr, waves)
    return tr


def fwd_staged_trace(waves, spw, tokens):
    """The withdrawn second forward variant as described: the four-slab forward (mf32_fwd_kernel, s_red
    only, :216 and :301-308) with each slab's x staged in the wave's slab rows the way the pipelined
    backward stages it (:874-881) and read back as the lane's own rows, before and after the barrier."""
    tr = Trace(waves, {"slab": waves * SLAB * 2, "s_red": 2 * 16 * 4})
    for it in range(tokens):
        for w in range(waves):
            for _ in range(spw):
                _stage_slab(tr, w, parts=(0,))
                _read_own_rows(tr, w, 0)
        _rms_sums(tr, waves, it, 1, 16)
        for w in range(waves):
            for _ in range(spw):
                _read_own_rows(tr, w, 0)
    return tr


def fwd_loop_trace(waves, spw, tokens, layer_wide):
    """mf32_fwd_loop_kernel: lane group 0 writes each of the wave's slabs' y at s_y[(slab 16 + r) 8 .. +8]
    before the RMS barrier and every lane group reads its slab's row back after it (:465-469, :483-485);
    dynamic LDS S 16 8 floats (:1880); layer-wide split operands staged by wave 0 (:423-435)."""
    S = waves * spw
    tr = Trace(waves, {"s_y": S * 16 * 8 * 4, "s_red": 2 * 16 * 4, "s_aa": 3 * 64 * 16})
    if layer_wide:
        _params_by_wave0(tr, "s_aa", 3 * 64 * 16, waves)
    for it in range(tokens):
        for w in range(waves):
            for s in range(spw):
                slab = w * spw + s
                tr.instr("s_y", w, "W", [(ln, 4 * (slab * 16 + r) * 8, 32) for ln, q, r in LANES if q == 0])
        _rms_sums(tr, waves, it, 1, 16)
        for w in range(waves):
            for s in range(spw):
                slab = w * spw + s
                tr.instr("s_y", w, "R", [(ln, 4 * (slab * 16 + r) * 8, 32) for ln, q, r in LANES])
    return tr


# ---------------------------------------------------------------------------------------------------
# launch shapes the host code chooses (mfma32.hip:1995-2024, :1870-1880)
# ---------------------------------------------------------------------------------------------------

def bwd_shapes():
    """(waves, slabs per wave (3 standing for 3 and more), pipelined) over C = 128 S up to 8192."""
    out = set()
    for S in range(1, 65):
        if S <= MAXW:
            out.add((S, 1, False))
            continue
        for spw in range(2, K["kMf32MaxSpw"] + 1):
            if S % spw == 0 and S // spw <= MAXW:
                pipe = spw <= K["kMf32PipeMaxSpw"] and S <= K["kMf32PipeMaxS"]
                out.add((S // spw, min(spw, 3), False))
                if pipe:
                    out.add((S // spw, min(spw, 3), True))
    return sorted(out)


@pytest.mark.parametrize("waves,spw,pipe", bwd_shapes())
def test_backward_slabs_are_private_and_synchronised(waves, spw, pipe):
    tr = bwd_trace(waves, spw, tokens=3, pipe=pipe)
    assert check(tr)
    # the staging rows of waves w and w + 4 (one SIMD) never meet: each wave's slab accesses before the
    # final reduction stay inside [w kMf32Slab, (w + 1) kMf32Slab) halfwords
    last = max(r[6] for r in tr.rows)
    for r in tr.rows:
        if r[0] == "slab" and r[6] < last - 1:
            assert r[3] * SLAB * 2 <= r[1] and r[2] <= (r[3] + 1) * SLAB * 2, r


@pytest.mark.parametrize("waves,spw", [(w, s) for w in range(1, MAXW + 1) for s in (1, 2)])
def test_withdrawn_staged_forward_layout_is_private(waves, spw):
    assert check(fwd_staged_trace(waves, spw, tokens=3), private=("slab",))


@pytest.mark.parametrize("waves,spw", [(w, s) for w in range(1, MAXW + 1) for s in (1, 2, 3, 16)
                                       if w * s * 128 <= K["kMf32FwdMaxC"]])
@pytest.mark.parametrize("layer_wide", [False, True])
def test_loop_forward_y_is_private_and_synchronised(waves, spw, layer_wide):
    assert check(fwd_loop_trace(waves, spw, tokens=3, layer_wide=layer_wide), private=("s_y",))


def test_the_model_catches_planted_mistakes():
    """The checker itself: a slab base of (wave % 4) kMf32Slab (waves w and w + 4 sharing rows), a
    cross-wave read with the barrier removed, and an access past the array all fail."""
    tr = Trace(8, {"slab": 8 * SLAB * 2})
    for w in range(8):
        base = (w % 4) * SLAB
        tr.instr("slab", w, "W", [(ln, 2 * (base + 8 * q * ROW + 8 * r), 16) for ln, q, r in LANES])
    with pytest.raises(AssertionError, match="per-wave array shared"):
        check(tr, private=("slab",))
    tr = Trace(2, {"s_red": 2 * 16 * 4})
    tr.instr("s_red", 0, "W", [(0, 0, 4)])
    tr.instr("s_red", 1, "R", [(5, 0, 4)])  # no barrier in between
    with pytest.raises(AssertionError, match="without a barrier"):
        check(tr)
    tr = Trace(1, {"s_y": 64})
    tr.instr("s_y", 0, "W", [(0, 60, 8)])
    with pytest.raises(AssertionError, match="out of bounds"):
        check(tr)
    # the RMS sums with one buffer instead of two: the next token's write of a wave's slot falls in the
    # epoch in which the other waves still read this token's slots, so it fails where [it & 1] passes
    tr = Trace(2, {"s_red": 2 * 16 * 4})
    for it in range(2):
        for w in range(2):
            tr.instr("s_red", w, "W", [(0, 4 * w, 4)])  # slot [0][w] for every token
        tr.barrier()
        for w in range(2):
            for src in range(2):
                tr.instr("s_red", w, "R", [(ln, 4 * src, 4) for ln in range(64)])
    with pytest.raises(AssertionError, match="without a barrier"):
        check(tr)
