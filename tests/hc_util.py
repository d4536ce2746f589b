"""Seeded hyper-connection read inputs (src/hc.cuh HcArgs) shared by the oracle and GPU tests."""
import numpy as np


def hc_inputs(N, HC, LR, T, seed, inject=True):
    """(weights as plain arrays, R, bo, inj_prev): Q8S matrices with int8 values and f16 scales ~ 0.02 / 127 (so dequantized
    weights ~ N(0, 0.02) in size), w_norm ~ 1 + 0.1 N(0, 1), bf16 inject rows, R ~ N(0, 1) per stream"""
    rng = np.random.default_rng(seed)
    D = HC * N
    q = lambda r, c: rng.integers(-127, 128, size=(r, c), dtype=np.int64).astype(np.int8)
    s = lambda r, c: (rng.uniform(0.5, 1.5, size=(r, c)) * 0.02 / 64).astype(np.float16).view(np.uint16)
    w = dict(N=N, HC=HC, LR=LR,
             w_norm=(1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
             dq=q(LR, D), dd=s(LR, D // 32), uq=q(D, LR), ud=s(D, LR // 32),
             w_inj=((0.02 * rng.standard_normal((HC, D))).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
             if inject else None)
    R = rng.standard_normal((T, D)).astype(np.float32)
    bo = rng.standard_normal((T, N)).astype(np.float32)
    inj = rng.standard_normal((T, HC)).astype(np.float32)
    return w, R, bo, inj


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def bf16(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)


def round_away(x):
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def q8_blocks(x):
    """int8 per 32 with float d = amax / 127 (hc.cuh q8_block), as float64 values d q, and q, d"""
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    d = (amax.astype(np.float32) / np.float32(127)).astype(np.float64)
    q = np.where(amax[:, None] == 0, 0, round_away(b / np.where(d == 0, 1, d)[:, None]))
    return (q * d[:, None]).reshape(-1), q.reshape(-1), d


def hc_read_f64(w, R, bo, inj, eps=1e-6):
    """the read in float64 from its definition: returns mixed, inject, R', the slices' partial dots and square sums"""
    N, HC, LR = w["N"], w["HC"], w["LR"]
    D, NS = HC * N, HC * N // 512
    T = R.shape[0]
    sig = lambda x: 1 / (1 + np.exp(-x))
    Rp = R.astype(np.float64).copy()
    if bo is not None:
        for c in range(HC):
            Rp[:, c * N:(c + 1) * N] += bo * 2 * sig(inj[:, c:c + 1] / HC)
    Wd = w["dq"].astype(np.float64) * np.repeat(f16(w["dd"]), 32, axis=1)
    Wu = w["uq"].astype(np.float64) * np.repeat(f16(w["ud"]), 32, axis=1)
    Wi = bf16(w["w_inj"]) if w["w_inj"] is not None else None
    mixed = np.empty((T, N))
    inject = np.zeros((T, HC))
    part = np.zeros((T, NS, LR + HC))
    ssp = np.empty((T, NS))
    for t in range(T):
        xs = Rp[t] * w["w_norm"]
        xv, _, _ = q8_blocks(xs.astype(np.float32).astype(np.float64))
        for s in range(NS):
            sl = slice(512 * s, 512 * (s + 1))
            ssp[t, s] = (Rp[t, sl] ** 2).sum()
            part[t, s, :LR] = Wd[:, sl] @ xv[sl]
            if Wi is not None:
                part[t, s, LR:] = Wi[:, sl] @ xs[sl]
        rs = 1 / np.sqrt(ssp[t].reshape(HC, -1).sum(axis=1) / N + eps)
        comb = (part[t].reshape(HC, -1, LR + HC).sum(axis=1) * rs[:, None]).sum(axis=0)
        lo = comb[:LR] / HC
        lo = lo * sig(lo)
        inject[t] = comb[LR:]
        lv, _, _ = q8_blocks(lo)
        g = (Wu @ lv).reshape(HC, N)
        mixed[t] = (sig(g) * (Rp[t] * w["w_norm"]).reshape(HC, N) * rs[:, None]).mean(axis=0)
    return mixed, inject, Rp, part, ssp
