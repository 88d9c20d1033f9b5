"""Writes tests/golden/attention_small.npz: small paged-attention problems
with their expected outputs, computed by the textbook definition in plain
Python loops (float64), independently of oracle/ and of the kernels.

    python tests/golden/make_attention_golden.py

Semantics (pagedattn.forward, kernels/pagedattn/pagedattn.cu:182-207,
:315-329, :418-446 of the reference): query row i of a sequence with q_len
query tokens and kv_len keys sits at position kv_len - q_len + i and sees
keys j <= that position (bottom-right causal); scale 1/sqrt(D); a row with no
visible key outputs 0 with lse = +inf; lse is natural-log logsumexp of the
scaled scores. Query head h reads KV head h // (Hq / Hkv).

Inputs are rounded to bfloat16-representable values so the same fixture
checks the fp32 and the bf16 kernels (the bf16 kernels see exactly these
inputs). Physical blocks are a seeded permutation and every slot no sequence
owns holds 1e3, so a wrong gather shows.
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    # decode: one query per sequence, 16 query heads per KV head, D 64 (the
    # shape of the MFMA decode kernel), contexts across block boundaries
    "decode_g16_d64": dict(q_lens=[1, 1, 1, 1, 1], kv_lens=[1, 17, 96, 200, 33],
                           hq=16, hkv=1, d=64, bs=16, seed=11),
    # decode with 32 heads per KV head and D 128
    "decode_g32_d128": dict(q_lens=[1, 1, 1], kv_lens=[70, 129, 5], hq=32, hkv=1, d=128,
                            bs=16, seed=12),
    # mixed prefill / decode with GQA (2 KV heads) and an empty context
    "mixed_gqa": dict(q_lens=[3, 1, 2, 1], kv_lens=[7, 0, 20, 9], hq=4, hkv=2, d=32, bs=8,
                      seed=13),
}


def bf16_round(x):
    """Round float64 -> nearest bfloat16 (ties to even), returned as float64."""
    f = x.astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def build(q_lens, kv_lens, hq, hkv, d, bs, seed):
    rng = np.random.default_rng(seed)
    nblk = [max(1, math.ceil(kv / bs)) for kv in kv_lens]
    nb = sum(nblk) + 3
    k_pool = np.full((nb, bs, hkv, d), 1e3)
    v_pool = np.full((nb, bs, hkv, d), 1e3)
    perm = rng.permutation(np.arange(1, nb))  # block 0 stays unowned
    table = np.zeros((len(q_lens), max(nblk)), dtype=np.int32)
    dense, cur = [], 0
    for s, kv in enumerate(kv_lens):
        ids = perm[cur:cur + nblk[s]]
        cur += nblk[s]
        table[s, :nblk[s]] = ids
        k = bf16_round(rng.standard_normal((kv, hkv, d)))
        v = bf16_round(rng.standard_normal((kv, hkv, d)))
        dense.append((k, v))
        for j in range(kv):
            k_pool[ids[j // bs], j % bs] = k[j]
            v_pool[ids[j // bs], j % bs] = v[j]
    q = bf16_round(rng.standard_normal((sum(q_lens), hq, d)))
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return q, k_pool, v_pool, table, np.asarray(kv_lens, dtype=np.int32), qsl, dense


def textbook(q, dense, q_lens, kv_lens, qsl, hq, hkv, d):
    scale = 1.0 / math.sqrt(d)
    out = np.zeros_like(q)
    lse = np.full(q.shape[:2], np.inf)
    for s, (ql, kv) in enumerate(zip(q_lens, kv_lens)):
        k, v = dense[s]
        for i in range(ql):
            row = int(qsl[s]) + i
            last = kv - ql + i
            for h in range(hq):
                g = h // (hq // hkv)
                keys = list(range(0, min(kv, last + 1)))
                if not keys:
                    continue
                sc = []
                for j in keys:
                    acc = 0.0
                    for t in range(d):
                        acc += float(q[row, h, t]) * float(k[j, g, t])
                    sc.append(acc * scale)
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                z = sum(w)
                for t in range(d):
                    acc = 0.0
                    for wj, j in zip(w, keys):
                        acc += wj * float(v[j, g, t])
                    out[row, h, t] = acc / z
                lse[row, h] = m + math.log(z)
    return out, lse


def main():
    arrays = {}
    for name, c in CASES.items():
        q, kp, vp, table, lens, qsl, dense = build(**c)
        out, lse = textbook(q, dense, c["q_lens"], c["kv_lens"], qsl, c["hq"], c["hkv"], c["d"])
        arrays.update({f"{name}/q": q, f"{name}/k_pool": kp, f"{name}/v_pool": vp,
                       f"{name}/block_table": table, f"{name}/seq_lens": lens,
                       f"{name}/query_start_loc": qsl, f"{name}/out": out, f"{name}/lse": lse,
                       f"{name}/shape": np.asarray([c["hq"], c["hkv"], c["d"], c["bs"],
                                                    max(c["q_lens"])], dtype=np.int32)})
    path = os.path.join(HERE, "attention_small.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {', '.join(CASES)}")


if __name__ == "__main__":
    main()
