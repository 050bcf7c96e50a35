"""kitty_append_tokens through the C-ABI against a numpy model of the
documented routing (kitty_hip.h; the FP16 part of the reference's
KittyInferencePipeline.push_token, kitty/pipeline.py:115-181): each
sequence's token goes to its sink while the sink holds fewer than S tokens,
else to its key / value buffer rows; a full, unspilled buffer sets
overflow[b] and writes nothing; an out-of-range slot is skipped.  Rows are
compared bit for bit, and every buffer row the model does not write must keep
its old contents.

Cases: the production row (H x D = 8 x 128, the kernel's preloaded 2 x 64
16-byte vectors), one vector per row (H=1, D=8), a row past the preloaded
vectors (4 x 512), no sink, values sharing the key buffer's counter, and
strided key / value rows.
"""
import ctypes

import numpy as np
import pytest
import torch

from kitty import _hip


def _model(slots, key, value, sk, sv, bk, bv, vb, fill, qlen, vlen, S, T, V, own):
    ov = np.zeros(len(slots), np.int32)
    for i, s in enumerate(slots):
        if not 0 <= s < len(fill):
            continue
        f, q = fill[s], qlen[s]
        v = vlen[s] if own else q
        if f < S:
            sk[s, :, f], sv[s, :, f] = key[i], value[i]
            fill[s] += 1
        elif q >= T or (own and v >= V):
            ov[i] = 1
        else:
            bk[s, :, q] = key[i]
            if own:
                vb[s, :, v] = value[i]
                vlen[s] += 1
            else:
                bv[s, :, q] = value[i]
            qlen[s] += 1
    return ov


def _layout(t):
    return _hip.SlotLayout(t.stride(0), t.stride(1), t.stride(2))


@pytest.mark.gpu
@pytest.mark.parametrize("H,D,S,own,pad", [
    (8, 128, 4, True, 0),    # production row: 128 vectors, all preloaded
    (8, 128, 4, False, 0),   # values share buf_len and buf_v
    (1, 8, 4, True, 0),      # one 16-byte vector per token
    (4, 512, 4, True, 0),    # 256 vectors: half through the tail loop
    (2, 64, 0, True, 0),     # no sink (NULL sink buffers)
    (8, 128, 2, True, 16),   # key / value rows strided inside a wider tensor
])
def test_append_matches_model(H, D, S, own, pad):
    dev = "cuda:0"
    g = torch.Generator().manual_seed(H * 1000 + D + S)
    NS, T, V = 6, 5, 7
    # slot states: sink not full, buffer with room, key buffer full, value
    # buffer full, last free buffer row; slots -1 and NS are out of range
    fill = np.array([S // 2, S, S, S, S, S], np.int32)
    qlen = np.array([0, 2, T, 1, T - 1, 0], np.int32)
    vlen = np.array([0, 3, 2, V, V - 1, 0], np.int32)
    if not own:
        vlen = qlen.copy()
    slots = np.array([3, 0, -1, 1, 4, NS, 2], np.int32)
    B = len(slots)

    def rnd(*shape):
        return torch.randn(*shape, generator=g).half()

    wide_k, wide_v = rnd(B, H, D + pad), rnd(B, H, D + pad)
    key, value = wide_k[..., :D], wide_v[..., :D]
    sk, sv = rnd(NS, H, max(S, 1), D), rnd(NS, H, max(S, 1), D)
    bk, bv, vb = rnd(NS, H, T, D), rnd(NS, H, T, D), rnd(NS, H, V, D)

    exp = [t.numpy().view(np.int16).copy() for t in (sk, sv, bk, bv, vb)]
    efill, eqlen, evlen = fill.copy(), qlen.copy(), vlen.copy()
    eov = _model(slots, key.numpy().view(np.int16), value.numpy().view(np.int16), *exp, efill, eqlen, evlen,
                 S, T, V, own)

    d = {n: t.to(dev) for n, t in dict(wk=wide_k, wv=wide_v, sk=sk, sv=sv, bk=bk, bv=bv, vb=vb).items()}
    dk, dv = d["wk"][..., :D], d["wv"][..., :D]
    c = {n: torch.from_numpy(x).to(dev) for n, x in dict(fill=fill, qlen=qlen, vlen=vlen, slots=slots).items()}
    ov = torch.zeros(B, dtype=torch.int32, device=dev)

    a = _hip.AppendArgs()
    a.key, a.value = dk.data_ptr(), dv.data_ptr()
    a.key_s_seq, a.key_s_head, a.value_s_seq, a.value_s_head = dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1)
    a.slots = c["slots"].data_ptr()
    if S:
        a.sink_k, a.sink_v = d["sk"].data_ptr(), d["sv"].data_ptr()
    a.sink_layout = _layout(d["sk"])
    a.buf_k, a.buf_v = d["bk"].data_ptr(), d["bv"].data_ptr()
    a.buf_layout = _layout(d["bk"])
    a.sink_fill, a.buf_len, a.overflow = c["fill"].data_ptr(), c["qlen"].data_ptr(), ov.data_ptr()
    a.batch, a.num_kv_heads, a.head_dim, a.sink_size, a.buf_tokens, a.num_slots = B, H, D, S, T, NS
    if own:
        a.val_len, a.val_buf, a.val_tokens = c["vlen"].data_ptr(), d["vb"].data_ptr(), V
        a.val_layout = _layout(d["vb"])
    _hip.check(_hip.load().kitty_append_tokens(ctypes.byref(a), _hip.stream_ptr(torch.device(dev))))
    torch.cuda.synchronize()

    got = [d[n].cpu().numpy().view(np.int16) for n in ("sk", "sv", "bk", "bv", "vb")]
    for name, e, r in zip(("sink_k", "sink_v", "buf_k", "buf_v", "val_buf"), exp, got):
        assert np.array_equal(e, r), name
    assert np.array_equal(c["fill"].cpu().numpy(), efill)
    assert np.array_equal(c["qlen"].cpu().numpy(), eqlen)
    if own:
        assert np.array_equal(c["vlen"].cpu().numpy(), evlen)
    assert np.array_equal(ov.cpu().numpy(), eov)
    assert eov.tolist() == [int(own), 0, 0, 0, 0, 0, 1]   # value-full slot 3 (own values), key-full slot 2
    # the append leaves its source rows (and their pad columns) unchanged
    assert np.array_equal(d["wk"].cpu().numpy().view(np.int16), wide_k.numpy().view(np.int16))


@pytest.mark.parametrize("s_head", [-128, 1 << 28])
def test_append_rejects_head_strides_beyond_32bit_offsets(s_head):
    """The kernel addresses one token's H x D block of a buffer with 32-bit
    byte offsets; a negative or oversized head stride is refused before any
    device work (the pointers below are never dereferenced)."""
    L = _hip.load()
    a = _hip.AppendArgs()
    fake = 1 << 20
    a.key = a.value = a.slots = a.buf_k = a.buf_v = a.sink_fill = a.buf_len = a.overflow = fake
    a.key_s_seq, a.key_s_head, a.value_s_seq, a.value_s_head = 8 * 128, 128, 8 * 128, 128
    a.buf_layout = _hip.SlotLayout(8 * 16 * 128, s_head, 128)
    a.batch, a.num_kv_heads, a.head_dim, a.sink_size, a.buf_tokens, a.num_slots = 1, 8, 128, 0, 16, 1
    rc = L.kitty_append_tokens(ctypes.byref(a), None)
    assert rc == _hip.KITTY_E_INVALID
    assert b"head stride" in L.kitty_last_error()
