"""Shared inputs of the tiled NVFP4 GEMM tests: random records in the form of the reference's
own test (crates/oominf-cuda/tests/moe_tiled.rs:45-99: scale_2 as float 0, codes at byte
64, one e4m3 scale byte per 16 inputs between about 2^-2 and 2^2), token rows, and the f64
evaluation that test checks against (moe_tiled.rs:176-214)."""
import numpy as np

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def e4m3_f64(b):
    b = np.asarray(b, dtype=np.int64)
    e, m = (b >> 3) & 15, (b & 7).astype(np.float64)
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    return np.where(b & 0x80, -v, v)


class Records:
    def __init__(self, rng, experts, n, k):
        self.n, self.k, self.w_off = n, k, 64
        self.s_off = self.w_off + n * k // 2
        self.stride = (self.s_off + n * k // 16 + 4095) // 4096 * 4096
        self.recs = []
        for _ in range(experts):
            r = np.zeros(self.stride, dtype=np.uint8)
            r[:4] = np.array([0.01 + 0.02 * abs(rng.uniform(-1, 1))], dtype=np.float32).view(np.uint8)
            r[self.w_off:self.s_off] = rng.integers(0, 256, self.s_off - self.w_off, dtype=np.uint8)
            r[self.s_off:self.s_off + n * k // 16] = 0x28 + rng.integers(0, 0x28, n * k // 16, dtype=np.uint8)
            self.recs.append(r)

    def weights_f64(self, e):
        """[n, k] f64: e2m1(code) * e4m3(scale) * scale_2, exactly."""
        r = self.recs[e]
        codes = r[self.w_off:self.s_off].reshape(self.n, self.k // 2)
        c = np.empty((self.n, self.k), dtype=np.int64)
        c[:, 0::2], c[:, 1::2] = codes & 15, codes >> 4
        sc = e4m3_f64(r[self.s_off:self.s_off + self.n * self.k // 16]).reshape(self.n, self.k // 16)
        s2 = float(r[:4].view(np.float32)[0])
        return E2M1[c] * np.repeat(sc, 16, axis=1) * s2


def bf16_round(x):
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x7fff + ((b >> 16) & 1)) & 0xffff0000).astype(np.uint32)).view(np.float32)


def case(n, k, counts, seed, tokens=64):
    rng = np.random.default_rng(seed)
    recs = Records(rng, len(counts), n, k)
    x = (2.0 * rng.uniform(-1, 1, (tokens, k))).astype(np.float32)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    rows = rng.integers(0, tokens, int(off[-1]), dtype=np.int32)
    return recs, x, off, rows


def f64_eval(recs, x, off, rows, exact):
    """(y [A, n] f64, sum |x w| [A, n]) with x rounded to bf16 unless exact."""
    xv = x.astype(np.float64) if exact else bf16_round(x).astype(np.float64)
    A = int(off[-1])
    y = np.zeros((A, recs.n))
    mag = np.zeros((A, recs.n))
    for e in range(len(recs.recs)):
        a0, a1 = int(off[e]), int(off[e + 1])
        if a1 == a0:
            continue
        w = recs.weights_f64(e)
        xe = xv[rows[a0:a1]]
        y[a0:a1] = xe @ w.T
        mag[a0:a1] = np.abs(xe) @ np.abs(w).T
    return y, mag


SHAPES = [(200, 96, [1, 0, 37, 70]), (640, 2560, [3, 33, 64]), (2560, 640, [17, 40])]
