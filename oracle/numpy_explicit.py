"""Independent NumPy restatement with a hand-derived backward (test infrastructure).

Forward follows ``flashrnn/flashrnn2/reference.py:74-114`` (the same cell
formulas as ``torch_restatement``) and the operand policy of
``flashrnn/flashrnn2/torch_backend.py:53-58``. Backward is written out by
hand from those formulas -- it is *not* autograd -- so that comparing it with
the autograd restatement pins both: a dropped term, a wrong sign or a
transposed operand in either one shows up as a mismatch.

The backward here is the one the HIP kernels implement:

* ``dry`` (the cotangent of ``R h``) per cell, below;
* ``dh_{t-1} += round(R^T dry)`` and ``dR += round(dry^T h_{t-1})`` where
  ``round`` is the BF16 round trip of the ``fp32_state_bf16_mma`` policy
  (identity for the mathematical policy);
* torch tie rules: ``maximum(a, b)`` sends half the cotangent to each input
  on a tie; ``where`` sends all of it to the selected input.

BF16 rounding is round-to-nearest-even by bit manipulation on FP32. FP16
rounding (``operands="f16"``: the same policy with FP16 operands, FlashRNN2's
FP16 contract of ``flashrnn/flashrnn2/state_contract.py:21-49``) is NumPy's own
float16 conversion, independent of torch's.
"""

from __future__ import annotations

import numpy as np

SIZES = {"lstm": (4, 4, 2), "slstm": (4, 4, 4), "gru": (3, 4, 1), "elman": (1, 1, 1)}


def bf16_round(x: np.ndarray) -> np.ndarray:
    """FP32 -> BF16 (round to nearest, ties to even) -> FP32. NaN stays NaN."""
    x32 = np.ascontiguousarray(x, dtype=np.float32)
    bits = x32.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x32), x32, out)


def f16_round(x: np.ndarray) -> np.ndarray:
    """FP32 -> FP16 (NumPy's round to nearest even) -> FP32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def _rounder(bf16_operands, operands):
    if operands is None:
        operands = "bf16" if bf16_operands else None
    return {None: lambda a: a, "bf16": bf16_round, "f16": f16_round}[operands]


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _logsig(x):
    return np.minimum(x, 0) - np.log1p(np.exp(-np.abs(x)))


def forward(wx, R, b, s0, cell, bf16_operands=False, operands=None):
    """Returns (history [S,B,T,N,D], caches). Arrays in their given float dtype.
    ``operands``: None, "bf16" or "f16" (``bf16_operands=True`` means "bf16")."""
    dt = wx.dtype.type
    B, T, _, N, D = wx.shape
    rnd = _rounder(bf16_operands, operands)
    Rr = rnd(R).astype(dt)
    state = s0[:, :, 0].copy()
    hist, caches = [], []
    zero_start = cell == "slstm" and bool(np.all(state[2] == 0))
    for t in range(T):
        x = wx[:, t]
        hh = rnd(state[0]).astype(dt)
        ry = np.einsum("bnp,gnop->bgno", hh, Rr)
        cache = {"hh": hh, "old": state}
        if cell == "elman":
            h = np.tanh(x[:, 0] + ry[:, 0] + b[0])
            new = h[None]
            cache["h"] = h
        elif cell == "gru":
            cand = ry[:, 0] + b[0]
            r = _sig(x[:, 0] + ry[:, 1] + b[1])
            u = _sig(x[:, 1] + ry[:, 2] + b[2])
            v = np.tanh(x[:, 2] + b[3] + r * cand)
            new = (u * state[0] + (1 - u) * v)[None]
            cache.update(cand=cand, r=r, u=u, v=v)
        else:
            g = x + ry + b
            gi, gf, gz, go = g[:, 0], g[:, 1], g[:, 2], g[:, 3]
            if cell == "lstm":
                si, sf, tz, so = _sig(gi), _sig(gf), np.tanh(gz), _sig(go)
                c = sf * state[1] + si * tz
                tc = np.tanh(c)
                new = np.stack((so * tc, c))
                cache.update(si=si, sf=sf, tz=tz, so=so, tc=tc)
            else:
                lf = _logsig(gf) + state[3]
                zero = zero_start and t == 0
                m = gi if zero else np.maximum(gi, lf)
                ia, fa = np.exp(gi - m), np.exp(lf - m)
                tz, so = np.tanh(gz), _sig(go)
                c = fa * state[1] + ia * tz
                npre = fa * state[2] + ia
                n = np.maximum(npre, 1)
                new = np.stack((so * c / n, c, n, m))
                cache.update(gi=gi, gf=gf, lf=lf, m=m, zero=zero, ia=ia, fa=fa, tz=tz,
                             so=so, c=c, npre=npre, n=n)
        state = new.astype(dt)
        hist.append(state)
        caches.append(cache)
    return np.stack(hist, axis=2), caches


def _tie_weights(a, b):
    """Cotangent share of ``a`` in ``maximum(a, b)`` (torch rule)."""
    return np.where(a > b, 1.0, np.where(a == b, 0.5, 0.0))


def backward(wx, R, b, s0, cell, d_hist, d_last, bf16_operands=False, operands=None):
    """Explicit backward. ``d_hist`` [S,B,T,N,D], ``d_last`` [S,B,1,N,D].

    Returns (dwx, dR, db, ds0) with the same shapes as the inputs.
    """
    dt = wx.dtype.type
    B, T, _, N, D = wx.shape
    rnd = _rounder(bf16_operands, operands)
    Rr = rnd(R).astype(dt)
    _, caches = forward(wx, R, b, s0, cell, bf16_operands, operands)
    S = s0.shape[0]
    dwx = np.zeros_like(wx)
    dR = np.zeros_like(R)
    db = np.zeros_like(b)
    carry = d_last[:, :, 0].copy()  # cotangent of the state after the last step
    for t in reversed(range(T)):
        cache = caches[t]
        ds = carry + d_hist[:, :, t]
        old = cache["old"]
        nxt = np.zeros_like(ds)  # cotangent of state t-1 (direct paths)
        if cell == "elman":
            da = ds[0] * (1 - cache["h"] ** 2)
            dry = da[:, None]
            dwx[:, t, 0] = da
            db[0] += da.sum(0)
        elif cell == "gru":
            dh = ds[0]
            r, u, v, cand = cache["r"], cache["u"], cache["v"], cache["cand"]
            du = dh * (old[0] - v)
            dv = dh * (1 - u)
            nxt[0] = dh * u
            dva = dv * (1 - v * v)
            dcand = dva * r
            dra = dva * cand * r * (1 - r)
            dua = du * u * (1 - u)
            dry = np.stack((dcand, dra, dua), axis=1)
            dwx[:, t] = np.stack((dra, dua, dva), axis=1)
            db += np.stack((dcand, dra, dua, dva)).sum(1)
        elif cell == "lstm":
            dh, dc = ds[0], ds[1]
            si, sf, tz, so, tc = (cache[k] for k in ("si", "sf", "tz", "so", "tc"))
            dgo = dh * tc * so * (1 - so)
            dc = dc + dh * so * (1 - tc * tc)
            dgi = dc * tz * si * (1 - si)
            dgf = dc * old[1] * sf * (1 - sf)
            dgz = dc * si * (1 - tz * tz)
            nxt[1] = dc * sf
            dry = np.stack((dgi, dgf, dgz, dgo), axis=1)
            dwx[:, t] = dry
            db += dry.sum(0)
        else:
            dh, dc, dn, dm = ds
            k = cache
            so, c, n = k["so"], k["c"], k["n"]
            dgo = dh * c / n * so * (1 - so)
            dc = dc + dh * so / n
            dn = dn - dh * so * c / (n * n)
            dnpre = dn * _tie_weights(k["npre"], np.ones_like(n))
            dfa = dc * old[1] + dnpre * old[2]
            dia = dc * k["tz"] + dnpre
            nxt[1] = dc * k["fa"]
            nxt[2] = dnpre * k["fa"]
            dgz = dc * k["ia"] * (1 - k["tz"] ** 2)
            dgi = dia * k["ia"]
            dlf = dfa * k["fa"]
            dm = dm - dia * k["ia"] - dfa * k["fa"]
            if k["zero"]:
                dgi = dgi + dm
            else:
                w = _tie_weights(k["gi"], k["lf"])
                dgi = dgi + dm * w
                dlf = dlf + dm * (1 - w)
            nxt[3] = dlf
            dgf = dlf * _sig(-k["gf"])
            dry = np.stack((dgi, dgf, dgz, dgo), axis=1)
            dwx[:, t] = dry
            db += dry.sum(0)
        dhh = np.einsum("bgno,gnop->bnp", dry, Rr)
        nxt[0] = nxt[0] + rnd(dhh.astype(dt)).astype(dt)
        dR += rnd(np.einsum("bgno,bnp->gnop", dry, cache["hh"]).astype(dt)).astype(dt)
        carry = nxt.astype(dt)
    ds0 = carry[:, :, None]
    assert ds0.shape == (S, B, 1, N, D)
    return dwx, dR, db, ds0
