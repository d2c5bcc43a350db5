"""CPU oracle for the fused 4-bit dequant-GEMV path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this module, and only as the checker (or, for the CPU baseline, as the
thing timed on the host).  The product package never imports it: its packers are
native C++ in ``libfourbit.so`` and its decode/GEMV runs in HIP kernels.

This is a plain numpy / torch-CPU restatement of the path's arithmetic, written for
clarity, not speed.  Every function states the reference code it follows or, where
the reference has no counterpart (GF4, E2M1, FWHT and nibble packing do not exist in
jvap2/If_I_could_turn_back_time), the published algorithm it restates.  How each
function is pinned (closed forms, brute force, the reference's own known-answer
test, scipy) is listed in its docstring and implemented in ``tests/test_oracle.py``.

Canonical formats (build decisions, fixed by the golden fixtures under
``tests/golden/``):

* weights ``[N, K]`` (out x in), K contiguous;
* canonical codes ``uint8 [N, K/2]``: byte ``j`` of a row holds element ``2j`` in
  bits 3:0 and element ``2j+1`` in bits 7:4;
* GF4 codebook ``uint16 [N, K/128, 16]`` (fp16 bit patterns, non-decreasing);
* E2M1 scales ``uint8 [N, K/32]`` (E8M0: value ``2**(s-127)``).
"""
from __future__ import annotations

import numpy as np
import torch

GF4_GROUP = 128
E2M1_GROUP = 32
GF4_LEVELS = 16

# E2M1 magnitudes by 3-bit index (OCP Microscaling Formats v1.0, section 5.3.3).
E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float64)


# --------------------------------------------------------------------------------------
# Jenks natural breaks with k classes (GF4 codebooks)
# --------------------------------------------------------------------------------------
def jenks_ssd_table(v_sorted: np.ndarray):
    """Within-class sum of squared deviations for every class [i, j) of sorted rows.

    ``v_sorted``: float64 ``[G, n]``.  Returns ``(ssd [G, n+1, n+1], S1 [G, n+1])``
    with ``ssd[g, i, j] = (S2[j]-S2[i]) - (S1[j]-S1[i])**2 / (j-i)`` for ``i < j``
    (+inf elsewhere), where S1/S2 are sequential fp64 prefix sums.

    Follows the reference's Jenks cost (``cuda_helpers.py:151-184``: per split index,
    left SSD + right SSD of a sorted array) generalised from 2 to k classes, written
    with prefix sums (Fisher 1958).
    """
    G, n = v_sorted.shape
    S1 = np.zeros((G, n + 1), np.float64)
    S2 = np.zeros((G, n + 1), np.float64)
    np.cumsum(v_sorted, axis=1, out=S1[:, 1:])  # sequential left-to-right accumulate
    np.cumsum(v_sorted * v_sorted, axis=1, out=S2[:, 1:])
    i = np.arange(n + 1)[:, None]
    j = np.arange(n + 1)[None, :]
    cnt = (j - i).astype(np.float64)
    valid = j > i
    cnt = np.where(valid, cnt, 1.0)
    s = S1[:, None, :] - S1[:, :, None]          # [G, i, j] = S1[j] - S1[i]
    q = S2[:, None, :] - S2[:, :, None]
    ssd = q - (s * s) / cnt
    ssd = np.where(valid[None], ssd, np.inf)
    return ssd, S1


def jenks_breaks(v_sorted: np.ndarray, k: int):
    """Optimal k-class contiguous partition of each sorted row (Fisher/Jenks DP).

    Returns ``(bounds [G, k+1] int64, cost [G] float64)``: class c covers sorted
    positions ``[bounds[c], bounds[c+1])``; every class is non-empty.  Recurrence
    ``D[m][j] = min_{m-1 <= i < j} D[m-1][i] + SSD(i, j)``; ties resolve to the
    smallest break index ``i`` (``np.argmin`` returns the first minimum).  For
    ``k = 2`` this is the reference's rule: argmin over split index of left-SSD +
    right-SSD (``cuda_helpers.py:151-184`` kernel, argmin at ``:386-389``).
    """
    G, n = v_sorted.shape
    if not 1 <= k <= n:
        raise ValueError("need 1 <= k <= n")
    ssd, _ = jenks_ssd_table(v_sorted)
    D = ssd[:, 0, :].copy()                       # one class: [0, j)
    back = np.zeros((k + 1, G, n + 1), np.int64)
    for m in range(2, k + 1):
        cand = D[:, :, None] + ssd                # [G, i, j]
        idx = np.arange(n + 1)
        cand[:, idx < m - 1, :] = np.inf          # first m-1 classes need >= m-1 points
        arg = np.argmin(cand, axis=1)             # first minimum -> smallest i
        Dn = np.take_along_axis(cand, arg[:, None, :], axis=1)[:, 0, :]
        Dn[:, : m] = np.inf                       # m classes need j >= m
        D = Dn
        back[m] = arg
    bounds = np.zeros((G, k + 1), np.int64)
    bounds[:, k] = n
    j = np.full(G, n, np.int64)
    for m in range(k, 1, -1):
        i = back[m, np.arange(G), j]
        bounds[:, m - 1] = i
        j = i
    return bounds, D[:, n]


def jenks2(values: np.ndarray):
    """Two-class natural breaks over a whole array, the reference's pruning rule
    (``Linear_Mask`` / ``Bias_Mask``, ``cuda_helpers.py:378-411``, over the kernels at
    ``:85-118`` and ``:151-184``): for every split ``idx`` in ``[0, n)`` of the ascending
    values, the SSD of ``[0, idx)`` about its mean plus the SSD of ``[idx, n)`` about its
    own (``idx = 0`` is one class: "no split"); the first argmin is the split; the values at
    sorted positions ``>= split`` are kept; ``GVF = (ssd(0) - ssd(split)) / (ssd(0) + 1e-8)``.

    Unlike ``jenks_breaks(v, 2)``, whose DP forces two non-empty classes, split 0 is a
    candidate here, as in the reference (its argmin runs over every idx); a constant array
    therefore keeps everything.  The sums follow the build's fixed fp64 order (stable
    ascending sort with -0.0 == +0.0; centre c = sorted[n // 2]; prefix sums sequential in
    blocks of 256, block totals sequential in superblocks of 256 blocks, superblock totals
    sequential), so that the native versions can be compared bit for bit.  Returns
    ``(keep bool [n], split, gvf, ssd [n])``."""
    w = np.asarray(values, dtype=np.float32).reshape(-1)
    n = w.size
    if n < 1 or not np.isfinite(w).all():
        raise ValueError("need a non-empty finite array")
    order = np.argsort(w, kind="stable")          # -0.0 == +0.0 under <
    ssd = jenks2_ssd(w[order])
    split = int(np.argmin(ssd))                               # first minimum
    keep = np.zeros(n, bool)
    keep[order[split:]] = True
    gvf = (ssd[0] - ssd[split]) / (ssd[0] + 1e-8)
    return keep, split, float(gvf), ssd


def jenks2_ssd(srt: np.ndarray) -> np.ndarray:
    """The within-class SSD of every split ``idx`` in ``[0, n)`` of an array taken in the
    order given (the caller sorts it), float64 ``[n]``: what the reference's
    ``jenks_optimization_cuda`` / ``jenks_optimization_biases_cuda`` return per split
    (``cuda_helpers.py:151-211``, ``:85-146``): class ``[0, idx)`` about its mean plus class
    ``[idx, n)`` about its own, ``idx = 0`` being one class.  float32 or float64 values
    (float64 ones are used as they are); the sums in the build's fixed fp64 order (centre
    c = srt[n // 2]; prefix sums sequential in blocks of 256, block totals sequential in
    superblocks of 256 blocks, superblock totals sequential):
    ``ssd(i) = [i ? Q(i) - P(i)^2 / i : 0] + [(Qt - Q(i)) - (Pt - P(i))^2 / (n - i)]``."""
    srt = np.asarray(srt).reshape(-1)
    if srt.dtype not in (np.float32, np.float64):
        srt = srt.astype(np.float32)
    n = srt.size
    if n < 1:
        raise ValueError("need a non-empty array")
    c = np.float64(srt[n // 2])
    d = srt.astype(np.float64) - c
    q = d * d
    blk, sup = 256, 256
    nblk = -(-n // blk)
    nsup = -(-nblk // sup)

    def blocked(v):
        pad = np.zeros(nblk * blk)
        pad[:n] = v
        loc = np.cumsum(pad.reshape(nblk, blk), axis=1)       # sequential within a block
        lx = np.concatenate([np.zeros((nblk, 1)), loc[:, :-1]], axis=1).reshape(-1)[:n]
        tot = loc[:, -1]                                      # block totals
        tpad = np.zeros(nsup * sup)
        tpad[:nblk] = tot
        bl = np.cumsum(tpad.reshape(nsup, sup), axis=1)
        bx = np.concatenate([np.zeros((nsup, 1)), bl[:, :-1]], axis=1).reshape(-1)[:nblk]
        u = bl[:, -1]
        sx = np.concatenate([[0.0], np.cumsum(u)])           # sx[nsup] = total
        i = np.arange(n)
        b = i // blk
        return (sx[b // sup] + bx[b]) + lx, sx[nsup]

    P, Pt = blocked(d)
    Q, Qt = blocked(q)
    i = np.arange(n, dtype=np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        left = np.where(i == 0, 0.0, Q - (P * P) / i)
    rp = Pt - P
    right = (Qt - Q) - (rp * rp) / (n - i)
    return left + right


def jenks2_filters(w: np.ndarray):
    """The reference's ``Conv_Mask`` (``cuda_helpers.py:333-376``) over its per-filter kernel
    (``:219-255``): the two-class rule of ``jenks2`` on every filter on its own, a filter being
    one (out, in) slice of an ``[out, in, kh, kw]`` weight (``flat = w.view(out * in, -1)``,
    sorted per row, ``min(dim=2)`` per filter).  ``w`` is ``[nf, n]``; returns ``(keep bool
    [nf, n], split int [nf], gvf float [nf])``."""
    w = np.asarray(w, dtype=np.float32)
    nf, n = w.shape
    keep = np.zeros((nf, n), bool)
    split = np.zeros(nf, np.int64)
    gvf = np.zeros(nf, np.float64)
    for f in range(nf):
        keep[f], split[f], gvf[f], _ = jenks2(w[f])
    return keep, split, gvf


def f64_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """fp64 -> fp32 -> fp16, each step round-to-nearest-even; returns uint16 bits."""
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16).view(np.uint16)


def gf4_quantize(w: np.ndarray, group: int = GF4_GROUP, k: int = GF4_LEVELS):
    """GF4: per (row, group) Jenks-16 codebook + 4-bit codes.

    ``w`` float32 ``[N, K]``.  Returns ``(codes uint8 [N, K] (unpacked), codebook
    uint16 [N, K/group, 16])``.  Per group: stable sort (value, then index), the
    k-class DP above, centroid = (S1[j]-S1[i])/(j-i) in fp64 rounded fp64->fp32->fp16,
    code = class index in ascending order.
    """
    w = np.asarray(w, np.float32)
    N, K = w.shape
    if K % group:
        raise ValueError("K must be a multiple of the group size")
    G = K // group
    vals = w.reshape(N * G, group).astype(np.float64)
    if not np.isfinite(vals).all():
        raise ValueError("weights must be finite")
    order = np.argsort(vals, axis=1, kind="stable")
    vs = np.take_along_axis(vals, order, axis=1)
    codes = np.empty((N * G, group), np.uint8)
    books = np.empty((N * G, k), np.uint16)
    chunk = 512
    for c0 in range(0, N * G, chunk):
        sl = slice(c0, min(c0 + chunk, N * G))
        bounds, _ = jenks_breaks(vs[sl], k)
        S1 = np.zeros((vs[sl].shape[0], group + 1), np.float64)
        np.cumsum(vs[sl], axis=1, out=S1[:, 1:])
        lo, hi = bounds[:, :-1], bounds[:, 1:]
        mean = (np.take_along_axis(S1, hi, 1) - np.take_along_axis(S1, lo, 1)) / (hi - lo)
        books[sl] = f64_to_f16_bits(mean)
        pos = np.arange(group)[None, :]
        cls = (pos[:, :, None] >= bounds[:, None, 1:-1]).sum(-1)  # class of sorted position
        cs = np.empty_like(cls)
        np.put_along_axis(cs, order[sl], cls, axis=1)
        codes[sl] = cs.astype(np.uint8)
    return codes.reshape(N, K), books.reshape(N, G, k)


def gf4_quantize_masked(w: np.ndarray, keep: np.ndarray, group: int = GF4_GROUP):
    """GF4 with a keep mask: masked weights decode to exactly 0.

    The reference multiplies the dequantized weight by its mask (``layers.py:37``,
    ``:43``), so pruned weights stay exactly zero; plain Jenks-16 can put zeros in a
    class with a non-zero mean.  Per group with at least one masked entry: Jenks with
    ``min(15, kept)`` classes over the kept values (stable-sorted, as
    ``gf4_quantize``), an exact-zero entry inserted after the strictly negative
    centroids, the rest of the 16 entries repeating the last used one; masked codes
    point at the zero entry.  Groups with nothing masked are ``gf4_quantize``'s.
    Group-by-group loop (test sizes only).
    """
    w = np.asarray(w, np.float32)
    keep = np.asarray(keep) != 0
    N, K = w.shape
    G = K // group
    codes = np.zeros((N, K), np.uint8)
    books = np.zeros((N, G, 16), np.uint16)
    full = keep.reshape(N, G, group).all(-1)
    if full.any():
        c, b = gf4_quantize(w.reshape(N, G, group)[full], group)
        codes.reshape(N, G, group)[full] = c
        books[full] = b[:, 0]
    for n in range(N):
        for g in range(G):
            sl = slice(g * group, (g + 1) * group)
            kp = keep[n, sl]
            if kp.all():
                continue
            vals = w[n, sl][kp].astype(np.float64)
            m = vals.size
            k = min(15, m)
            book = np.zeros(16, np.uint16)
            c = np.zeros(group, np.uint8)
            if k:
                order = np.argsort(vals, kind="stable")
                vs = vals[order]
                bounds, _ = jenks_breaks(vs[None], k)
                bounds = bounds[0]
                S1 = np.concatenate([[0.0], np.cumsum(vs)])
                cb = f64_to_f16_bits(
                    (S1[bounds[1:]] - S1[bounds[:-1]]) / (bounds[1:] - bounds[:-1]))
                cls_sorted = (np.arange(m)[:, None] >= bounds[None, 1:-1]).sum(-1)
                cls = np.empty(m, np.int64)
                cls[order] = cls_sorted
                z = int((cb.view(np.float16).astype(np.float64) < 0).sum())
                book[:z] = cb[:z]
                book[z] = 0
                book[z + 1:k + 1] = cb[z:]
                book[k + 1:] = book[k]
                c[:] = z
                c[np.flatnonzero(kp)] = cls + (cls >= z)
            codes[n, sl] = c
            books[n, g] = book
    return codes, books


def gf4_dequant(codes: np.ndarray, codebook: np.ndarray, group: int = GF4_GROUP) -> np.ndarray:
    """w[n,k] = codebook[n, k/group, code[n,k]] as fp16 bits (uint16 [N, K])."""
    N, K = codes.shape
    g = np.arange(K) // group
    return codebook[np.arange(N)[:, None], g[None, :], codes.astype(np.int64)]


# --------------------------------------------------------------------------------------
# E2M1 with E8M0 group scales (MXFP4-style)
# --------------------------------------------------------------------------------------
def e2m1_round_index(q: np.ndarray) -> np.ndarray:
    """Round |q| (float64) onto E2M1_GRID: nearest, ties to the even index, saturating
    at 6.  Returns the 3-bit magnitude index."""
    a = np.abs(np.asarray(q, np.float64))
    # midpoints between consecutive grid values
    mids = (E2M1_GRID[:-1] + E2M1_GRID[1:]) / 2.0
    idx = np.searchsorted(mids, a, side="left")        # a <= mid -> lower index
    tie = np.isin(a, mids)
    # at a tie searchsorted(left) gives the lower index; move to the even one
    up = tie & (idx % 2 == 1)
    idx = idx + up
    return np.minimum(idx, 7).astype(np.uint8)


def e8m0_exponent(amax: np.ndarray) -> np.ndarray:
    """Shared exponent e = floor(log2 amax) - 2 (OCP MX v1.0 section 6.3), clamped to the
    E8M0 range [-127, 127]; amax == 0 gives e = 0 (scale byte 127)."""
    amax = np.asarray(amax, np.float64)
    m, ex = np.frexp(amax)                  # amax = m * 2**ex, m in [0.5, 1)
    e = ex.astype(np.int64) - 1 - 2
    e = np.where(amax == 0, 0, e)
    return np.clip(e, -127, 127)


def e2m1_quantize(w: np.ndarray, group: int = E2M1_GROUP):
    """Returns ``(codes uint8 [N, K] unpacked, scales uint8 [N, K/group])``.

    code = sign<<3 | index(RNE(|w| / 2**e)), sign = signbit(w) (so -0.0 -> code 8).
    """
    w = np.asarray(w, np.float32)
    N, K = w.shape
    if K % group:
        raise ValueError("K must be a multiple of the group size")
    if not np.isfinite(w).all():
        raise ValueError("weights must be finite")
    G = K // group
    wg = w.reshape(N, G, group).astype(np.float64)
    e = e8m0_exponent(np.abs(wg).max(-1))
    q = wg / np.exp2(e)[..., None]
    idx = e2m1_round_index(q)
    sign = np.signbit(wg).astype(np.uint8)
    codes = (sign << 3) | idx
    return codes.reshape(N, K).astype(np.uint8), (e + 127).astype(np.uint8)


def e2m1_decode_code(codes: np.ndarray) -> np.ndarray:
    """E2M1 code -> float32 value (code 8 is -0.0)."""
    c = np.asarray(codes, np.int64)
    mag = E2M1_GRID[c & 7]
    return np.where(c & 8, -mag, mag).astype(np.float32)


def e2m1_dequant(codes: np.ndarray, scales: np.ndarray, group: int = E2M1_GROUP) -> np.ndarray:
    """w = E2M1(code) * 2**(scale-127), exact in float32 (float32 [N, K])."""
    N, K = codes.shape
    g = np.arange(K) // group
    e = scales.astype(np.int64)[:, g] - 127
    return np.ldexp(e2m1_decode_code(codes).astype(np.float64), e).astype(np.float32)


# --------------------------------------------------------------------------------------
# Activations as two MX-E4M3 terms (the B operand of the native FP4 MFMA path)
# --------------------------------------------------------------------------------------
E4M3_MAX = 448.0
MX_BLOCK = 32


def e4m3_round(v: np.ndarray):
    """Round |v| <= 448 (float64) to OCP E4M3 (e4m3fn: exponent bias 7, 3 fraction bits,
    subnormal step 2**-9, largest finite 448), nearest with ties to even.  Returns
    ``(codes uint8, values float64)``; the sign bit follows signbit(v).  No counterpart in
    the reference (OCP 8-bit Floating Point Specification v1.0, E4M3)."""
    v = np.asarray(v, np.float64)
    a = np.abs(v)
    if (a > E4M3_MAX).any():
        raise ValueError("e4m3_round takes |v| <= 448")
    _, ex = np.frexp(a)                          # a = m 2**ex, m in [0.5, 1)
    e = np.maximum(ex.astype(np.int64) - 1, -6)  # binade; below 2**-6 the subnormal step
    step = np.ldexp(1.0, e - 3)
    r = np.round(a / step) * step                # np.round: half to even
    _, ex2 = np.frexp(r)
    e2 = np.where(r >= 2.0 ** -6, ex2.astype(np.int64) - 1, -7)  # -7: subnormal / zero
    frac = np.where(e2 >= -6, r / np.ldexp(1.0, e2) - 1.0, r / 2.0 ** -9 / 8.0)
    code = ((e2 + 7) << 3) | np.round(frac * 8).astype(np.int64)
    code = np.where(r == 0, 0, code) | (np.signbit(v).astype(np.int64) << 7)
    return code.astype(np.uint8), np.where(np.signbit(v), -r, r)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """E4M3 code -> float64 (codes 0x7F / 0xFF are NaN)."""
    c = np.asarray(codes, np.int64)
    e, m = (c >> 3) & 15, c & 7
    mag = np.where(e > 0, np.ldexp(1.0 + m / 8.0, e - 7), np.ldexp(m / 8.0, -6))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return np.where(c & 0x80, -mag, mag)


def mx_exponent(amax: np.ndarray) -> np.ndarray:
    """The smallest e with amax <= 448 * 2**e, clamped to the E8M0 range [-127, 127];
    amax == 0 gives -127.  (Unlike OCP MX's floor(log2 amax) - 8, no value saturates.)"""
    amax = np.asarray(amax, np.float64)
    m, ex = np.frexp(amax)
    e = ex.astype(np.int64) - 9 + (m > 0.875)
    return np.clip(np.where(amax > 0, e, -127), -127, 127)


def mx_split_x(x, terms: int = 2):
    """x [B, K] (float values, e.g. bf16) -> ``(codes uint8 [terms, B, K], scales uint8
    [terms, B, K/32])``.  Term t rounds to E4M3, per 32-value block with its own E8M0 scale
    2**mx_exponent(block max), what the earlier terms left of x (float64, exact).  The
    native FP4 path's split (fb_gemv_mx, fb_mx_split).  No counterpart in the reference."""
    x = np.asarray(x, np.float64)
    B, K = x.shape
    if K % MX_BLOCK:
        raise ValueError("K must be a multiple of 32")
    rem = x.reshape(B, K // MX_BLOCK, MX_BLOCK).copy()
    codes, scales = [], []
    for _ in range(terms):
        e = mx_exponent(np.abs(rem).max(-1))
        c, val = e4m3_round(np.ldexp(rem, -e[..., None]))
        rem = rem - np.ldexp(val, e[..., None])
        codes.append(c.reshape(B, K))
        scales.append((e + 127).astype(np.uint8))
    return np.stack(codes), np.stack(scales)


def mx_terms_value(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Sum of the terms of mx_split_x (float64 [B, K])."""
    T, B, K = codes.shape
    v = e4m3_decode(codes).reshape(T, B, K // MX_BLOCK, MX_BLOCK)
    e = scales.astype(np.int64)[..., None] - 127
    return np.ldexp(v, e).sum(0).reshape(B, K)


def y_ref_mx(codes, scales_w, x, terms: int = 2):
    """E2M1 W (exact decode) times the MX split of x, float64 [B, N]: what the native FP4
    MFMA computes, up to its fp32 accumulation."""
    W = e2m1_dequant(codes, scales_w).astype(np.float64)
    c, s = mx_split_x(np.asarray(x, np.float64), terms)
    return mx_terms_value(c, s) @ W.T


# --------------------------------------------------------------------------------------
# Nibble packing
# --------------------------------------------------------------------------------------
def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """uint8 [N, K] codes (0..15) -> uint8 [N, K/2]; element 2j low nibble, 2j+1 high."""
    c = np.asarray(codes, np.uint8)
    if (c > 15).any():
        raise ValueError("codes must be 4-bit")
    return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 2), np.uint8)
    out[:, 0::2] = p & 15
    out[:, 1::2] = p >> 4
    return out


# --------------------------------------------------------------------------------------
# Walsh-Hadamard transform (Sylvester order, normalised by 1/sqrt(b)), blockwise on rows
# --------------------------------------------------------------------------------------
def fwht_rows(a: np.ndarray, block: int) -> np.ndarray:
    """Normalised blockwise FWHT along the last axis, computed in float64.

    Iterative butterflies with stride h = 1, 2, 4, ..., block/2 (pair (u, u+h) ->
    (u+h', ...) = (a+b, a-b)), then a multiply by 1/sqrt(block).  For a row-vector
    block w this is ``w @ H_b / sqrt(b)`` (H symmetric), and for a column x it is
    ``H_b x / sqrt(b)``.
    """
    a = np.asarray(a, np.float64)
    K = a.shape[-1]
    if block & (block - 1) or K % block:
        raise ValueError("block must be a power of two dividing K")
    lead = a.shape[:-1]
    t = a.reshape(-1, K // block, block).copy()
    h = 1
    while h < block:
        t = t.reshape(t.shape[0], t.shape[1], block // (2 * h), 2, h)
        x, y = t[:, :, :, 0, :], t[:, :, :, 1, :]
        t = np.stack([x + y, x - y], axis=3).reshape(t.shape[0], t.shape[1], block)
        h *= 2
    t = t * (1.0 / np.sqrt(block))
    return t.reshape(*lead, K)


def rotate_weights(w: np.ndarray, block: int) -> np.ndarray:
    """Offline rotation W' = W @ H_b/sqrt(b) per K-block, fp64 then one RNE to fp32."""
    return fwht_rows(np.asarray(w, np.float32), block).astype(np.float32)


# --------------------------------------------------------------------------------------
# Dequantize-then-matmul (the reference's forward structure)
# --------------------------------------------------------------------------------------
def dequant_f32(fmt: str, codes, meta) -> torch.Tensor:
    """Dense fp32 [N, K] weight from unpacked codes + codebook/scales."""
    if fmt == "gf4":
        bits = gf4_dequant(codes, meta)
        return torch.from_numpy(bits.view(np.float16).astype(np.float32))
    if fmt == "e2m1":
        return torch.from_numpy(e2m1_dequant(codes, meta))
    raise ValueError(fmt)


def rotate_x(x: torch.Tensor, block: int) -> torch.Tensor:
    """x' = H x / sqrt(b) per block in fp64, returned as fp32."""
    return torch.from_numpy(fwht_rows(x.double().numpy(), block).astype(np.float32))


def y_ref(fmt: str, codes, meta, x: torch.Tensor, fwht_block: int = 0) -> torch.Tensor:
    """``F.linear(x.float(), dequant(W))`` on the CPU in fp32 -- the structure of
    ``Quantization_Experiments/layers.py:36-38`` (dequantize, then ``F.linear``) and
    ``brecq.py:323-329``.  With ``fwht_block`` the activation is rotated first."""
    W = dequant_f32(fmt, codes, meta)
    xf = x.float()
    if fwht_block:
        xf = rotate_x(xf, fwht_block)
    return torch.nn.functional.linear(xf, W)


# --------------------------------------------------------------------------------------
# The reference's own 4-bit format (QuantLinear.commit) as a GF4 codebook
# --------------------------------------------------------------------------------------
def quantlinear_commit_weight(w, theta, mask=None, bitwidth=4):
    """Restates ``Quantization_Experiments/layers.py:23-26`` (per-row scale and floor)
    and ``:39-45`` (commit): ``mask * s * round(Q + [sigmoid(Theta)*1.2-0.1 > 0.5])``
    with ``s = amax_k|w| / (2**(b-1)-1) + 1e-12`` and ``Q = floor(w / s)``; fp32 torch
    arithmetic as in the reference.  Returns (W_q, s, level) with level = Q_round."""
    w = torch.as_tensor(w, dtype=torch.float32)
    qmax = 2 ** (bitwidth - 1) - 1
    s = w.abs().amax(dim=1, keepdim=True) / qmax + 1e-12
    Q = torch.floor(w / s)
    th = (torch.sigmoid(torch.as_tensor(theta, dtype=torch.float32)) * 1.2 - 0.1 > 0.5).float()
    Qr = torch.round(Q + th)
    m = torch.ones_like(w) if mask is None else torch.as_tensor(mask, dtype=torch.float32)
    return m * s * Qr, s, Qr * (m != 0)


def levels_to_gf4(levels, scale, group: int = GF4_GROUP):
    """Integer-level weight ``scale[n] * level[n,k]`` as a GF4 codebook.

    Per group: ``lo = min level`` (+0.0 so a -0 minimum becomes +0), code = level - lo,
    ``codebook[j] = fp16_rne(fp32(scale[n] * (lo + min(j, hi - lo))))``.  Raises when a
    group spans more than 16 levels.  The weight it encodes is the reference's
    committed one, ``mask * s * Q_round`` (``layers.py:43``: fp32 product, then one
    rounding to fp16 here), and brecq's ``clamp(...) * delta`` (``brecq.py:88-92``).
    Returns ``(codes uint8 [N, K] unpacked, codebook uint16 [N, K/group, 16])``.
    """
    lv = np.asarray(levels, np.float32)
    sc = np.asarray(scale, np.float32).reshape(-1)
    N, K = lv.shape
    G = K // group
    lg = lv.reshape(N, G, group)
    if not np.isfinite(lg).all() or (np.floor(lg) != lg).any():
        raise ValueError("levels must be finite integers")
    lo = lg.min(-1) + np.float32(0.0)
    hi = lg.max(-1)
    if ((hi - lo) > 15).any():
        raise ValueError("a group spans more than 16 levels")
    j = np.arange(16, dtype=np.float32)
    lev = lo[..., None] + np.minimum(j[None, None, :], (hi - lo)[..., None])
    prod = (sc[:, None, None] * lev).astype(np.float32)
    book = prod.astype(np.float16).view(np.uint16)
    codes = (lg - lo[..., None]).astype(np.uint8).reshape(N, K)
    return codes, book


def adaround_hard_levels(W_floor, alpha, mask, qmin: int, qmax: int):
    """Integer levels of brecq's AdaRound quantizer with the rounding made hard.

    ``AdaRoundQuantizer.forward`` (``brecq.py:81-92``) returns
    ``clamp(mask * (W_floor + h), qmin, qmax) * delta`` with
    ``h = clip(sigmoid(alpha) * 1.2 - 0.1, 0, 1)``; the hard level rounds h as the
    reference's ``QuantLinear.commit`` rounds its Theta (``layers.py:41``: h > 0.5 -> 1).
    Where ``|alpha|`` saturates the clip, h is already 0 or 1 and the result equals the
    soft forward exactly.  fp32 torch arithmetic as in the reference.
    """
    Wf = torch.as_tensor(W_floor, dtype=torch.float32)
    a = torch.as_tensor(alpha, dtype=torch.float32)
    m = torch.as_tensor(mask, dtype=torch.float32)
    h = torch.clamp(torch.sigmoid(a) * 1.2 - 0.1, 0, 1)
    hard = (h > 0.5).float()
    return torch.clamp(m * (Wf + hard), qmin, qmax)
