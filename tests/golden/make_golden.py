"""Writes the golden fixtures in this directory (run from the repo root:
``python tests/golden/make_golden.py``).

Each fixture is a compressed .npz of inputs and expected outputs:

* known_answers.npz — the reference's two known-answer tests
  (tests/test_quantize.py:141-166: per-channel [0, 1, 2, 3] -> byte 0xE4,
  scale 1, zero 0; :247-268: a constant 3.0 value block -> codes 3, stored
  scale 0), written out by hand, not computed;
* quant_block.npz — one seeded 128 x 128 key block with 16 outlier channels
  (x8) and its INT4 ranks, one value block, and the oracle's packed pages;
* decode_small.npz — the reference unit-test shape (2 KV / 2 Q heads,
  D = 16, G = 8, D_boost = 4, 3 pages, 4 sinks, 5 tail tokens) and the
  production shape (2 KV / 8 Q heads, D = G = 128, D_boost = 16, 3 pages,
  32 sinks, 17 tail tokens): pools, queries, segments and the oracle output.

The oracle (oracle/) is pinned by tests/test_oracle.py; these files freeze
its outputs so a later change to either the oracle or the kernels shows up as
a fixture mismatch, and give the GPU box vectors that need no CPU oracle run.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def boost_row(D, d_boost, sentinel, channels):
    bi = np.full(D, sentinel, np.uint8)
    for r, c in enumerate(channels):
        bi[c] = r
    return bi


def known_answers():
    key = np.tile(np.array([0, 1, 2, 3], np.float16), (4, 1))              # (D=4, G=4)
    return dict(ka_key=key, ka_key_t2b=np.full((4, 1), 0xE4, np.uint8),
                ka_key_scale=np.ones(4, np.float16), ka_key_zero=np.zeros(4, np.float16),
                ka_value=np.full((8, 16), 3.0, np.float16), ka_value_packed=np.full((8, 4), 0xFF, np.uint8),
                ka_value_scale=np.zeros(8, np.float16), ka_value_zero=np.zeros(8, np.float16))


def quant_block(rng):
    D = G = 128
    dk, sentinel = 16, 17
    chans = rng.permutation(D)[:dk]
    bi = boost_row(D, dk, sentinel, chans)
    key = rng.standard_normal((G, D)).astype(np.float32)                    # token-major
    key[:, chans] *= 8.0
    key = key.astype(np.float16)
    value = rng.standard_normal((G, D)).astype(np.float16)
    t2b, th, s, z = O.quantize_key(key.T.copy(), bi, dk, sentinel)
    pk, sv, zv = O.quantize_value(value)
    return dict(key=key, value=value, boost_idx=bi, d_boost=np.int32(dk), sentinel=np.int32(sentinel),
                t2b=t2b, thigh=th, key_scale=s, key_zero=z, packed=pk, value_scale=sv, value_zero=zv)


def decode_case(rng, prefix, H, Hq, D, G, dk, n_pages, n_sink, n_tail):
    sentinel = dk + 1
    P = n_pages + 2
    kb = np.zeros((P, H, D, G // 4), np.uint8)
    kh = np.zeros((P, H, dk, G // 4), np.uint8)
    km = np.zeros((P, H, 2, D), np.float16)
    vp = np.zeros((P, H, G, D // 4), np.uint8)
    vm = np.zeros((P, H, G, 2), np.float16)
    bi = np.stack([boost_row(D, dk, sentinel, rng.permutation(D)[:dk]) for _ in range(H)])
    pages = rng.permutation(P)[:n_pages].astype(np.int32)
    for p in pages:
        for h in range(H):
            k = rng.standard_normal((D, G)).astype(np.float32)
            k[bi[h] < sentinel] *= 8.0
            kb[p, h], kh[p, h], km[p, h, 0], km[p, h, 1] = O.quantize_key(k.astype(np.float16), bi[h], dk, sentinel)
            vp[p, h], vm[p, h, :, 0], vm[p, h, :, 1] = O.quantize_value(rng.standard_normal((G, D)).astype(np.float16))
    q = rng.standard_normal((Hq, D)).astype(np.float16)
    sk = rng.standard_normal((H, n_sink, D)).astype(np.float16)
    sv = rng.standard_normal((H, n_sink, D)).astype(np.float16)
    tk = rng.standard_normal((H, n_tail, D)).astype(np.float16)
    tv = rng.standard_normal((H, n_tail, D)).astype(np.float16)
    out = O.paged_attention(q, pages, kb, kh, km, vp, vm, bi, dk, sk, sv, tk, tv, Hq, H, D)
    d = dict(q=q, pages=pages, kb=kb, kh=kh, km=km, vp=vp, vm=vm, bi=bi, d_boost=np.int32(dk), sk=sk, sv=sv,
             tk=tk, tv=tv, out=np.asarray(out, np.float32), shape=np.array([H, Hq, D, G], np.int32))
    return {f"{prefix}_{k}": v for k, v in d.items()}


def main():
    O.build()
    np.savez_compressed(os.path.join(HERE, "known_answers.npz"), **known_answers())
    np.savez_compressed(os.path.join(HERE, "quant_block.npz"), **quant_block(np.random.default_rng(2026)))
    rng = np.random.default_rng(7)
    cases = {}
    cases.update(decode_case(rng, "ref", 2, 2, 16, 8, 4, 3, 4, 5))
    cases.update(decode_case(rng, "prod", 2, 8, 128, 128, 16, 3, 32, 17))
    np.savez_compressed(os.path.join(HERE, "decode_small.npz"), **cases)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
