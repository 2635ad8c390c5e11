"""Needle tokens for full-size parity checks that can see missing work.

With random keys, attention over 10^5 or more tokens is a near-uniform average:
dropping a whole split, or a tenth of all tokens, moves the output by less than
the 2e-3 tolerance.  Needles fix that.  In every ``seg``-row segment of every
attended block, four rows become needles: the first row, the last row and two
random rows.  A needle's key points along the sum of its kv head's query heads.
Its score is then about ``target`` for every query head of the group, while
background scores stay O(1), so the needles carry all but ~1e-6 of the softmax
mass.  A needle's value is ``+-amp`` in one random dim and 0 elsewhere.
Dropping n of N needles moves an output dim by about n * amp / N.  A random
sign per needle keeps the output itself small, so the relative tolerance term
stays small too.

The check (``assert_sensitive_match``) is the contract tolerance (max-abs 2e-3,
rel 1e-2), plus lse at max-abs 2e-3 with no relative term, plus out at
norm-relative error 1e-2.  ``differs`` asks whether a result misses a reference
by more than ``margin`` times those bounds; negative controls use it against
the oracle with a block, a segment or a single needle removed.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import oracle as O

SCALE = 1 / math.sqrt(128)
THREADS = 16
ATOL, RTOL = 2e-3, 1e-2
LSE_ATOL = 2e-3
NORM_RTOL = 1e-2


def needle_rows(valid: np.ndarray, bt: int, rng: np.random.Generator, blocks=None, seg: int = 32, extra: int = 2):
    """(block ids, rows) of the needles: per ``seg``-row segment of every
    attended row range, the first and last row plus ``extra`` random rows
    (distinct).  ``blocks`` limits planting to those block ids (a selection)."""
    ids = range(len(valid)) if blocks is None else sorted(set(int(b) for b in blocks))
    out_b, out_t = [], []
    for b in ids:
        n = int(valid[b])
        n = max(0, min(bt, n if n >= 0 else bt + n))
        for s0 in range(0, n, seg):
            s1 = min(n, s0 + seg)
            rows = {s0, s1 - 1}
            span = np.arange(s0, s1)
            free = [r for r in span if r not in rows]
            if free:
                rows.update(int(r) for r in rng.choice(free, size=min(extra, len(free)), replace=False))
            for r in sorted(rows):
                out_b.append(b)
                out_t.append(r)
    return np.array(out_b, np.int64), np.array(out_t, np.int64)


def needle_keys(q: np.ndarray, kv_heads: int, scale: float, target: float = 10.0) -> np.ndarray:
    """[KVH, D] keys: kv head h's key is beta_h * unit(sum of its query heads),
    beta_h set so that the smallest score over the group is ``target``."""
    qh, d = q.shape
    gq = qh // kv_heads
    keys = np.zeros((kv_heads, d), np.float32)
    for h in range(kv_heads):
        grp = q[h * gq : (h + 1) * gq].astype(np.float64)
        u = grp.sum(axis=0)
        u /= np.linalg.norm(u)
        worst = float((grp @ u).min())
        assert worst > 0, "query heads of a group point apart; pick another seed"
        keys[h] = (target / (scale * worst)) * u
    return keys


def needle_values(n: int, kv_heads: int, d: int, amp: float, rng: np.random.Generator, run: int = 1) -> np.ndarray:
    """[n, KVH, D] values: +-amp in one random dim per (needle, kv head).
    ``run`` consecutive needles share the dim and the sign (``run`` = 4: the
    needles of one segment), so that dropping them moves one dim by
    run * amp / N instead of spreading amp / N over ``run`` dims."""
    v = np.zeros((n, kv_heads, d), np.float32)
    groups = -(-n // run)
    dims = np.repeat(rng.integers(0, d, (groups, kv_heads)), run, axis=0)[:n]
    signs = np.repeat(rng.choice([-1.0, 1.0], (groups, kv_heads)).astype(np.float32), run, axis=0)[:n]
    v[np.arange(n)[:, None], np.arange(kv_heads)[None, :], dims] = signs * amp
    return v


def plant(k4: np.ndarray, v4: np.ndarray, q: np.ndarray, valid: np.ndarray, scale: float, rng, *, amp: float,
          blocks=None, target: float = 10.0, seg: int = 32):
    """Overwrite the needle rows of float K/V [NB, BT, KVH, D] in place; returns (blocks, rows)."""
    nb, bt, kvh, d = k4.shape
    bb, tt = needle_rows(valid, bt, rng, blocks, seg)
    k4[bb, tt] = needle_keys(q, kvh, scale, target)[None]
    v4[bb, tt] = needle_values(len(bb), kvh, d, amp, rng)
    return bb, tt


def _errors(out, lse, ref_out, ref_lse):
    out, lse = np.asarray(out, np.float64), np.asarray(lse, np.float64)
    ref_out, ref_lse = np.asarray(ref_out, np.float64), np.asarray(ref_lse, np.float64)
    contract = np.max(np.abs(out - ref_out) - RTOL * np.abs(ref_out))
    contract_l = np.max(np.abs(lse - ref_lse) - RTOL * np.abs(ref_lse))
    lse_abs = np.max(np.abs(lse - ref_lse))
    norm_rel = np.linalg.norm(out - ref_out) / max(np.linalg.norm(ref_out), 1e-30)
    return contract, contract_l, lse_abs, norm_rel


def assert_sensitive_match(out, lse, ref_out, ref_lse, what: str = "") -> None:
    contract, contract_l, lse_abs, norm_rel = _errors(out, lse, ref_out, ref_lse)
    msg = f"{what}: out excess {contract:.3e}, lse excess {contract_l:.3e}, |dlse| {lse_abs:.3e}, norm-rel {norm_rel:.3e}"
    assert contract <= ATOL and contract_l <= ATOL, msg
    assert lse_abs <= LSE_ATOL, msg
    assert norm_rel <= NORM_RTOL, msg


def differs(out, lse, ref_out, ref_lse, margin: float = 2.0) -> bool:
    """True when (out, lse) misses the reference by more than ``margin`` times a bound of the check."""
    contract, contract_l, lse_abs, norm_rel = _errors(out, lse, ref_out, ref_lse)
    return bool(
        contract > margin * ATOL or contract_l > margin * ATOL or lse_abs > margin * LSE_ATOL
        or norm_rel > margin * NORM_RTOL
    )


def move_rows_to_end(arrays, block: int, rows) -> list[np.ndarray]:
    """Copies of [NB, BT, ...] arrays whose ``block`` has ``rows`` moved to its
    end, other rows kept in order: with that block's count reduced by
    len(rows), attention over the result is attention without those rows."""
    out = []
    for a in arrays:
        c = a.copy()
        bt = a.shape[1]
        keep = [r for r in range(bt) if r not in set(int(x) for x in rows)]
        c[block] = a[block][keep + [int(x) for x in rows]]
        out.append(c)
    return out


def half_kv(tokens: int, seed: int, value_scale: float, outliers: float, qh: int, kvh: int = 8):
    """fp16-representable K/V [T, KVH, 128] (float32) and an fp16 query, the workload recipes."""
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(tokens, kvh, 128, generator=gen, dtype=torch.float16).float() * value_scale
    v = torch.randn(tokens, kvh, 128, generator=gen, dtype=torch.float16).float() * value_scale
    q = torch.randn(qh, 128, generator=gen, dtype=torch.float16)
    if outliers:
        k[torch.rand(k.shape, generator=gen) < outliers] *= 8
        v[torch.rand(v.shape, generator=gen) < outliers] *= 8
    return q, k.numpy(), v.numpy()


def quantize(k: np.ndarray, v: np.ndarray, bits: int):
    k = k.astype(np.float16).astype(np.float32)
    v = v.astype(np.float16).astype(np.float32)
    pk, sk, valid = O.quantize_blocks(k, bits, 32, 128)
    pv, sv, _ = O.quantize_blocks(v, bits, 32, 128)
    return [pk, pv, sk, sv], valid


def needle_mass_share(q, pk, sk, bits, needles, lse) -> float:
    """Smallest share, over query heads, of the softmax mass the needles carry
    (their scores from the dequantised needle keys and the oracle's lse)."""
    bb, tt = needles
    qh = q.shape[0]
    kvh = pk.shape[2]
    gq = qh // kvh
    codes = O.unpack_np(pk[bb[0], tt[0]], bits, 128).astype(np.float64) - (1 << (bits - 1))
    keys = codes * np.repeat(sk[bb[0], tt[0]].astype(np.float64), 32, axis=-1)  # [KVH, D]
    shares = []
    for h in range(qh):
        s = SCALE * float(q[h].astype(np.float64) @ keys[h // gq])
        shares.append(math.exp(s + math.log(len(bb)) - float(lse[h])))
    return min(shares)


def oracle(q, arrays, valid, bits, table=None):
    pk, pv, sk, sv = arrays
    t = None if table is None else np.asarray(table, np.int32)
    return O.attention(q, pk, pv, sk, sv, valid, bits, 32, SCALE, block_table=t, threads=THREADS)


def controls(q, arrays, valid, bits, table, needles, single_needle=True):
    """Oracle results over the selection minus one full block, minus one
    32-token segment of another full block, and minus one needle row of a
    third (every occurrence of the dropped block leaves the selection)."""
    bt = arrays[0].shape[1]
    attended = list(range(len(valid))) if table is None else list(table)
    full = [b for b in attended if valid[b] == bt]
    out = {}
    drop = full[len(full) // 2]
    out["block"] = oracle(q, arrays, valid, bits, [b for b in attended if b != drop])
    b = full[len(full) // 3]
    seg = list(range(32, 64))
    v2 = valid.copy()
    v2[b] -= len(seg)
    out["segment"] = oracle(q, move_rows_to_end(arrays, b, seg), v2, bits, table)
    if single_needle:
        bb, tt = needles
        b = full[(2 * len(full)) // 3]
        row = int(tt[bb == b][3])
        v3 = valid.copy()
        v3[b] -= 1
        out["needle"] = oracle(q, move_rows_to_end(arrays, b, [row]), v3, bits, table)
    return out
