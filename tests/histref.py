"""Oracle decode outputs rebuilt from a raw token history, for the module
and pipeline tests (GPU and CPU).

``oracle_from_history`` cuts sinks, key pages, value pages and the FP16 key
and value tails out of the history from S, G and the value window R alone,
quantises the pages with the C oracle and attends them with the oracle's
decode, so it shares no bookkeeping with the pipeline under test.
"""
import numpy as np

import oracle as O


def oracle_from_history(K, V, q, S, G, bi, d_boost, sentinel, Hq, H, D, R=0):
    """Independent oracle: sinks / key pages / value pages / key and value
    tails cut from the raw token history (values of the last R tokens, and
    of the rest of their G-token block, stay FP16)."""
    T = K.shape[0]
    ns = min(S, T)
    npg = max(0, (T - S) // G)
    npv = max(0, T - S - R) // G
    P = max(npg, 1)
    kb = np.zeros((P, H, D, G // 4), np.uint8)
    kh = np.zeros((P, H, d_boost, G // 4), np.uint8)
    km = np.zeros((P, H, 2, D), np.float16)
    vp = np.zeros((P, H, G, D // 4), np.uint8)
    vm = np.zeros((P, H, G, 2), np.float16)
    for pi in range(npg):
        blk = slice(S + pi * G, S + (pi + 1) * G)
        for h in range(H):
            kb[pi, h], kh[pi, h], km[pi, h, 0], km[pi, h, 1] = O.quantize_key(K[blk, h].T.copy(), bi[h], d_boost,
                                                                               sentinel)
            vp[pi, h], vm[pi, h, :, 0], vm[pi, h, :, 1] = O.quantize_value(V[blk, h].copy())
    tail = slice(S + npg * G, T)
    if npv == npg:
        return O.paged_attention(q, np.arange(npg), kb, kh, km, vp, vm, bi, d_boost,
                                 K[:ns].transpose(1, 0, 2).copy(), V[:ns].transpose(1, 0, 2).copy(),
                                 K[tail].transpose(1, 0, 2).copy(), V[tail].transpose(1, 0, 2).copy(), Hq, H, D)
    vtail = slice(S + npv * G, T)
    return O.paged_attention_kv(q, np.arange(npg), np.arange(npv), kb, kh, km, vp, vm, bi, d_boost,
                                K[:ns].transpose(1, 0, 2).copy(), V[:ns].transpose(1, 0, 2).copy(),
                                K[tail].transpose(1, 0, 2).copy(), V[vtail].transpose(1, 0, 2).copy(), Hq, H, D)


def close(got, ref):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    assert np.isfinite(got).all()
    excess = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert (excess <= 0).all(), f"max |diff| {np.abs(got - ref).max():.3g}"
