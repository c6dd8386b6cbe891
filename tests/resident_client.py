"""Client side of the resident worker protocol (test infrastructure).

Restates the frame layouts the reference runtime reads
(ray_tracing/runtime/resident_runtime.py:41-44 hello, 110-114 request/reply,
116-162 prefill, 91-99 growth, 164-169 finish, 171-233 generation / stream replies,
235-250 vocabulary, 252-263 mlp, 265-305 attention, 358-379 resources, 386-389 end).
"""
import struct
import subprocess
import tempfile

import numpy as np


class Worker:
    def __init__(self, exe, asset_dir, capacity=300, env=None):
        self.stderr = tempfile.TemporaryFile()
        args = [str(exe), str(asset_dir / "optical_model.bin"), str(asset_dir / "vocabulary.bin"), str(capacity),
                "1", "rt_full", "0.08", "32", "8", "1", "4", "512", "8"]
        self.p = subprocess.Popen(args, stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=self.stderr, env=env)
        self.hello = struct.unpack("<5I", self.read(20))

    def read(self, n):
        parts = []
        while n:
            part = self.p.stdout.read(n)
            if not part:
                raise RuntimeError(self.error_text() or f"worker exited: {self.p.wait()}")
            parts.append(part)
            n -= len(part)
        return b"".join(parts)

    def error_text(self):
        self.stderr.seek(0)
        return self.stderr.read().decode("utf8", errors="replace")

    def request(self, op, count, debug=0, body=b""):
        self.p.stdin.write(struct.pack("<3I", op, count, int(debug)) + body)
        self.p.stdin.flush()
        status, size = struct.unpack("<2I", self.read(8))
        payload = self.read(size)
        if status:
            raise RuntimeError("Resident request failed")
        return payload

    def close(self):
        if self.p.poll() is None:
            try:
                self.p.stdin.write(struct.pack("<I", 0))
                self.p.stdin.flush()
            except OSError:
                pass
        code = self.p.wait(timeout=60)
        for s in (self.p.stdin, self.p.stdout):
            try:
                s.close()   # flushes what a dead worker never read
            except OSError:
                pass
        return code

    # op 6
    def mlp(self, x, layer, hidden, middle):
        x = np.ascontiguousarray(x, "<f4").reshape(-1, hidden)
        pay = self.request(6, len(x), layer, x.tobytes())
        n = len(x)
        size = n * (hidden + middle)
        v = np.frombuffer(pay, "<f4", count=size)
        out = dict(output=v[:n * hidden].reshape(n, hidden), activation=v[n * hidden:].reshape(n, middle),
                   feature_hits=np.frombuffer(pay, "<u4", count=n, offset=size * 4))
        off = size * 4 + n * 4
        out["times"] = np.frombuffer(pay, "<f8", count=3, offset=off)
        assert len(pay) == off + 24
        return out

    # op 4
    def vocabulary(self, q, hidden, vocab):
        pay = self.request(4, 1, 0, np.ascontiguousarray(q, "<f4").reshape(hidden).tobytes())
        off = 0

        def take(dtype, shape):
            nonlocal off
            a = np.frombuffer(pay, dtype, count=int(np.prod(shape)), offset=off).reshape(shape)
            off += a.nbytes
            return a

        blocks = hidden // 256
        r = dict(timings=take("<f8", (5,)), winner=take("<u4", (4,)), hit_count=int(take("<u4", (1,))[0]),
                 ids=take("<u4", (vocab,)), geometric_words=take("<f4", (256, hidden)),
                 query_packets=take("<u4", (blocks, 128, 2)), block_charts=take("<f4", (blocks, 4)),
                 block_hits=int(take("<u4", (1,))[0]))
        assert off == len(pay)
        return r

    # op 14
    def attention(self, q, k, v, gate, layer, query_start, history_start, heads, kv_heads, hd):
        q = np.ascontiguousarray(q, "<f4").reshape(-1, heads, hd)
        k = np.ascontiguousarray(k, "<f4").reshape(-1, kv_heads, hd)
        v = np.ascontiguousarray(v, "<f4").reshape(-1, kv_heads, hd)
        g = np.zeros_like(q) if gate is None else np.ascontiguousarray(gate, "<f4").reshape(q.shape)
        body = struct.pack("<4I", len(k), query_start, history_start, 0) + q.tobytes() + k.tobytes() + v.tobytes() + \
            g.tobytes()
        pay = self.request(14, len(q), layer, body)
        h = np.frombuffer(pay, "<u4", count=12)
        magic, rows, count, nh, nkv, dim, pb, block, stride, records, legacy, error = map(int, h)
        off = 80

        def take(dtype, shape):
            nonlocal off
            a = np.frombuffer(pay, dtype, count=int(np.prod(shape)), offset=off).reshape(shape)
            off += a.nbytes
            return a

        r = dict(magic=magic, rows=rows, count=count, heads=nh, kv_heads=nkv, dim=dim, packet_bytes=pb, block=block,
                 stride=stride, records=records, legacy=legacy, error=error,
                 timing=np.frombuffer(pay, "<f8", count=4, offset=48),
                 output=take("<f4", (rows, nh, dim)), physical=take("<f4", (rows, nh, 2)),
                 legacy_output=take("<f4", (rows, nh, dim)), legacy_physical=take("<f4", (rows, nh, 2)),
                 history_packets=take("u1", (count, pb)), receipts=take("<u4", (records, stride)))
        assert off == len(pay)
        return r

    # op 8
    def resources(self):
        return np.frombuffer(self.request(8, 0), "<u8")

    # op 1 / 11 / 12
    def prefill(self, ids, stops=(), checkpoint_tokens=None, boundaries=None, debug=0, hidden=0, depth=0):
        """debug 1 (layer capture) needs hidden and depth to read the captured rows."""
        ids = np.asarray(ids, "<u4")
        stop = list(stops)[:2] + [0xFFFFFFFF] * 2
        body = ids.tobytes() + struct.pack("<2I", *stop[:2])
        op = 1
        if checkpoint_tokens is not None:
            body += struct.pack("<I", checkpoint_tokens)
            op = 11
        if boundaries is not None:
            body += struct.pack("<I", len(boundaries)) + b"".join(struct.pack("<2I", p, k) for p, k in boundaries)
            op = 12
        pay = self.request(op, len(ids), debug, body)
        r = dict(times=np.frombuffer(pay, "<f8", count=6), control=np.frombuffer(pay, "<u4", count=8, offset=48))
        off = 80
        if debug == 1:   # resident_runtime.py:136-139
            n = len(ids) * hidden
            r["state"] = np.frombuffer(pay, "<f4", count=n, offset=off).reshape(len(ids), hidden)
            r["layers"] = np.frombuffer(pay, "<f4", count=depth * n, offset=off + 4 * n).reshape(depth, len(ids), hidden)
            off += 4 * n * (depth + 1)
        if len(pay) >= off + 32:
            r["footer"] = np.frombuffer(pay, "<u8", count=4, offset=off)
        return r

    PROFILE = ("projection_geometry", "bvh_update", "lens_history_trace", "coordinate_restore", "detector",
               "output_mlp", "vocabulary", "vocabulary_rt", "vocabulary_coefficients", "vocabulary_reduce")

    @staticmethod
    def generation(pay, profile=False, state=0):
        """A GenerationPacket reply (resident_runtime.py:190-233); state: hidden size of the
        debug-1 state that follows the hits."""
        r = dict(timing=np.frombuffer(pay, "<f8", count=18), control=np.frombuffer(pay, "<u4", count=8, offset=144))
        r["ids"] = np.frombuffer(pay, "<u4", count=64, offset=176)[:int(r["control"][1])].copy()
        r["hits"] = np.frombuffer(pay, "<u4", count=5, offset=432)
        off = 452
        if state:
            r["state"] = np.frombuffer(pay, "<f4", count=state, offset=off)
            off += 4 * state
        r["cache"] = np.frombuffer(pay, "<u4", count=4, offset=off + 32)
        if profile:
            r["profile"] = dict(zip(Worker.PROFILE, r["timing"][8:18]))
            r["detector"] = np.frombuffer(pay, "<f8", count=2, offset=off + 112)
        r["size"] = len(pay)
        assert len(pay) == off + 112 + (16 if profile else 0), len(pay)
        return r

    # op 2
    def generate(self, count, debug=0, hidden=0):
        return self.generation(self.request(2, count, debug), debug == 2, hidden if debug == 1 else 0)

    # op 9: one reply per token until the count or a stop
    def stream(self, count, debug=0):
        self.p.stdin.write(struct.pack("<3I", 9, count, debug))
        self.p.stdin.flush()
        out = []
        for _ in range(count):
            status, size = struct.unpack("<2I", self.read(8))
            pay = self.read(size)
            if status:
                raise RuntimeError("Resident stream failed")
            out.append(self.generation(pay, debug == 2))
            if not out[-1]["control"][2]:
                break
        return out

    # op 10
    def grow(self, capacity):
        return np.frombuffer(self.request(10, capacity), "<f8", count=3)

    # op 13
    def finish(self):
        pay = self.request(13, 0)
        return np.frombuffer(pay, "<u8", count=3), np.frombuffer(pay, "<f8", count=1, offset=24)
