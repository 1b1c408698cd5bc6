"""Writes synthetic exports in the format of the reference's converter (convert/export_engine.py:33-40,83-85) for the
loader tests: manifest.json + shard files, optionally in the packed "wire" form whose scale tensors are 8-bit log
codes (web/public/engine/wire.js:1-46), optionally with a lazy embedding (engine.js:113-172). Test infrastructure.

The wire code of a row of G f16 scales: m (f16 bits of the largest magnitude), j (u16), then per scale
sign << 7 | k with |scale| ~ m 2^(-k j / 4096); decode_scales restates the decoder's arithmetic: f64 product, rounded
to f32, then to f16, both to nearest even."""
import json
import math
import os

import numpy as np


def encode_scales(sc):
    """f16 [N][G] -> (header u8 [4N], codes u8 [N G])."""
    sc = np.asarray(sc, np.float16)
    N, G = sc.shape
    head = np.zeros((N, 2), np.uint16)
    codes = np.zeros((N, G), np.uint8)
    for r in range(N):
        a = np.abs(sc[r].astype(np.float64))
        m = a.max()
        head[r, 0] = np.float16(m).view(np.uint16)
        nz = a[a > 0]
        if m == 0 or len(nz) == 0:
            continue
        j = max(1, int(math.ceil(4096 * math.log2(m / nz.min()) / 127)))
        head[r, 1] = j
        for g in range(G):
            k = 127 if a[g] == 0 else min(127, max(0, int(round(4096 * math.log2(m / a[g]) / j))))
            codes[r, g] = (0x80 if sc[r, g] < 0 else 0) | k
    return head.view(np.uint8).reshape(-1), codes.reshape(-1)


def decode_scales(head, codes, N, G):
    """Inverse of the wire code: f16 [N][G]."""
    hd = np.asarray(head, np.uint8).view(np.uint16).reshape(N, 2)
    out = np.zeros((N, G), np.float16)
    cd = np.asarray(codes, np.uint8).reshape(N, G)
    for r in range(N):
        m = float(hd[r, 0:1].view(np.float16)[0])
        j = int(hd[r, 1])
        for g in range(G):
            c = int(cd[r, g])
            v = np.float16(np.float32(m * 2.0 ** (-(c & 127) * j / 4096)))
            out[r, g] = -v if c & 128 else v
    return out


def write_export(d, config, W, V, shard_limit=64 << 20, wire=False, lazy=None):
    """W: {name: (words u32 [N][K/32][4], scales f16 [N][K/32], N, K)} quantised tensors; V: {name: f32 array}.
    Returns the f16 scales the export carries, by tensor (decoded ones for a wire export)."""
    os.makedirs(d, exist_ok=True)
    items = []
    for name, (words, sc, N, K) in W.items():
        items.append((name + ".q", np.ascontiguousarray(words).view(np.uint8).reshape(N, K // 32, 16), {"N": N, "K": K}))
        items.append((name + ".s", np.ascontiguousarray(sc, np.float16), {}))
    for name, v in V.items():
        items.append((name, np.ascontiguousarray(v, np.float32), {}))
    index, blobs, off = {}, [], 0
    for name, arr, meta in items:
        pad = (-off) % 256
        if pad:
            blobs.append(b"\0" * pad)
            off += pad
        index[name] = {"offset": off, "bytes": arr.nbytes, "dtype": str(arr.dtype), "shape": list(arr.shape), **meta}
        blobs.append((name, arr.tobytes()))
        off += arr.nbytes
    shards, cur, start, pos = [], [], 0, 0
    for b in blobs:
        n = len(b[1]) if isinstance(b, tuple) else len(b)
        if cur and pos + n - start > shard_limit:
            shards.append((start, cur))
            cur, start = [], pos
        cur.append(b)
        pos += n
    shards.append((start, cur))
    scales = {k: v[1] for k, v in W.items()}
    entries = []
    for si, (s0, bs) in enumerate(shards):
        size = sum(len(b[1]) if isinstance(b, tuple) else len(b) for b in bs)
        if not wire:
            with open(os.path.join(d, "weights.%d.bin" % si), "wb") as f:
                for b in bs:
                    f.write(b[1] if isinstance(b, tuple) else b)
            entries.append({"path": "weights.%d.bin" % si, "start": s0, "bytes": size})
            continue
        wf = bytearray()
        for b in bs:
            if not isinstance(b, tuple):
                continue
            name, data = b
            t = index[name]
            t["wire"] = len(wf)
            if name.endswith(".s"):
                N, G = t["shape"]
                sc = np.frombuffer(data, np.float16).reshape(N, G)
                head, codes = encode_scales(sc)
                wf += head.tobytes() + codes.tobytes()
                t["u8"] = True
                scales[name[:-2]] = decode_scales(head, codes, N, G)
            else:
                wf += data
        with open(os.path.join(d, "wire.%d.bin" % si), "wb") as f:
            f.write(bytes(wf))
        entries.append({"path": "wire.%d.bin" % si, "start": s0, "bytes": size, "wire": True})
    manifest = {"config": config, "shards": entries, "tensors": index}
    if lazy is not None:
        manifest["embed"] = _write_lazy(d, W["embed"], **lazy)
    with open(os.path.join(d, "manifest.json"), "w") as f:
        json.dump(manifest, f)
    return scales


def _write_lazy(d, embed, bundled_ids, slots):
    words, sc, N, K = embed
    qb, sb = K // 2, K // 32 * 2
    rows = np.concatenate([np.ascontiguousarray(words).view(np.uint8).reshape(N, qb),
                           np.ascontiguousarray(sc, np.float16).view(np.uint8).reshape(N, sb)], axis=1)
    rows.tofile(os.path.join(d, "embed_rows.bin"))
    ids = np.asarray(bundled_ids, np.uint32)
    with open(os.path.join(d, "embed_bundle.bin"), "wb") as f:
        f.write(ids.tobytes() + rows[ids].tobytes())
    return {"bundle": "embed_bundle.bin", "rows": "embed_rows.bin", "bundled": len(ids), "vocab": N, "slots": slots,
            "parts": [["embed.q", qb], ["embed.s", sb]], "row_bytes": qb + sb}
