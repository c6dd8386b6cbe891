"""Checks of dense attention receipts (layout attention_receipts.hpp:16-29, compact false).

merge() combines the records of each (row, head) the way the reference's checker does
(verify_attention_receipts.py:172-184); bounds() asserts the record rules that checker
holds (verify_attention_receipts.py:146-171); compare() sets a device result against the
oracle's expected records."""
import numpy as np


def rows_heads(ctx_len, capacity, block, hq):
    """(row, head) of every record, in record order."""
    out = []
    for r, L in enumerate(ctx_len):
        active = max(0, min(int(L), capacity))
        for _ in range((active + block - 1) // block):
            out.extend((r, h) for h in range(hq))
    return out


def merge(m, z, u, index, rows, hq):
    """Records' (m, Z, U) merged per (row, head): (out, M, Z) of the whole history."""
    M = np.full((rows, hq), -np.inf)
    for (r, h), mi in zip(index, m):
        M[r, h] = max(M[r, h], float(mi))
    Z = np.zeros((rows, hq))
    U = np.zeros((rows, hq, u.shape[1]))
    for (r, h), mi, zi, ui in zip(index, m, z, u):
        s = np.exp(float(mi) - M[r, h])
        Z[r, h] += float(zi) * s
        U[r, h] += np.asarray(ui, np.float64) * s
    return U / Z[..., None], M, Z


def bounds(words, index, block):
    cov = block // 32
    for rec, (r, h) in zip(words, index):
        count = int(rec[2])
        assert 1 <= count <= block
        assert 1 <= int(rec[3]) <= count + (count + 3) // 4 - 1, ("exp evaluations", rec[3], count)
        assert 1 <= int(rec[4]) <= count, ("value runs", rec[4], count)
        assert int(rec[5]) == count
        assert int(rec[6]) == (2 + (count + 15) // 16 if h == 0 else 0)
        assert (int(rec[7]) & 3) == 3 and (int(rec[7]) & ~15) == 0
        assert bool(int(rec[7]) & 8) == (int(rec[4]) < count)
        want = [(1 << min(32, max(0, count - 32 * w))) - 1 for w in range(cov)]
        assert [int(x) for x in rec[8:8 + cov]] == want


def compare(raw, vals, words, tie, block, hd, label=""):
    """Device receipts raw [n, hd + 8 + block/32] (uint32) against the oracle's records."""
    raw = np.asarray(raw).view(np.uint32)
    cov = block // 32
    assert raw.shape == (len(vals), hd + 8 + cov), (label, raw.shape, len(vals))
    f = raw.view(np.float32)
    exact = ~tie
    # count, the traversal count and the coverage bits always; events where no near-tie
    np.testing.assert_array_equal(raw[:, [2, 5, 6]], words[:, [2, 5, 6]], err_msg=label)
    np.testing.assert_array_equal(raw[:, 8:8 + cov], words[:, 8:8 + cov], err_msg=label)
    np.testing.assert_array_equal(raw[exact][:, [3, 4, 7]], words[exact][:, [3, 4, 7]], err_msg=label)
    np.testing.assert_array_equal(raw[:, 4], words[:, 4], err_msg=label)   # value runs: exact decoded bits
    np.testing.assert_allclose(f[:, 0], vals[:, 0], rtol=1e-5, atol=1e-5, err_msg=label + " m")
    np.testing.assert_allclose(f[:, 1], vals[:, 1], rtol=1e-4, atol=1e-6, err_msg=label + " Z")
    u = f[:, 8 + cov:].astype(np.float64)
    scale = np.maximum(np.abs(vals[:, 3:]).max(1, keepdims=True), vals[:, 1:2])
    err = np.abs(u - vals[:, 3:]) / scale
    assert err.max() <= 2e-4, (label, "U", float(err.max()))
