"""Synthetic models and rows for the benchmark configurations.

Host preparation only (never timed): seeded weights and inputs, the
round-to-nearest quantizer that `tgc quantize` applies to these layers, and
TGIR text the backend (and the reference) load.

* rand(seed, scale): the reference's initializer (src/lower.c:661-668,
  :766-775): xorshift32 (13, 17, 5), seed 0 replaced by 0x9e3779b9,
  u = (x >> 8) / 2^24 in f32, value (2u - 1) * scale in f32. xorshift32 is
  linear over GF(2), so blocks of the stream are produced at once from
  precomputed powers of the step matrix.
* normal(seed, sigma): N(0, sigma) by Box-Muller over the same xorshift32
  stream (pairs u1 = ((x >> 8) + 1) / 2^24, u2 = (x >> 8) / 2^24, computed in
  f64, rounded to f32). The reference has no normal initializer; BASELINE's
  N(0, sigma) configs use this one.
* quantize_rtn: per-channel round-to-nearest with the MSE clip search of
  src/quant.c:176-200 (10 candidate scales amax (1 - 0.05 g) / lim, error
  summed in order, first strict minimum wins, codes nearbyint, scale stored
  as f32). GPTQ needs calibration activations and falls back to this for
  K > 2048 in the reference (src/quant.c:345-346), which is every quantized
  layer of configs 2 and 3 wider than 2048 inputs.
"""
import os

import numpy as np

_BLOCK = 4096
_POW = None


def _step(x):
    x = x ^ ((x << np.uint32(13)) & np.uint32(0xFFFFFFFF))
    x = x ^ (x >> np.uint32(17))
    x = x ^ ((x << np.uint32(5)) & np.uint32(0xFFFFFFFF))
    return x


def _powers():
    """cols[k, i] = step^(k+1)(1 << i) for k < _BLOCK: the columns of the
    GF(2) matrices of 1.._BLOCK xorshift steps."""
    global _POW
    if _POW is None:
        cols = np.empty((_BLOCK, 32), np.uint32)
        v = (np.uint32(1) << np.arange(32, dtype=np.uint32)).astype(np.uint32)
        for k in range(_BLOCK):
            v = _step(v)
            cols[k] = v
        _POW = cols
    return _POW


def _apply(cols, v):
    """GF(2) matrix (32 columns, uint32) times state(s) v."""
    v = np.asarray(v, np.uint32)
    acc = np.zeros(v.shape, np.uint32)
    for i in range(32):
        bit = (v >> np.uint32(i)) & np.uint32(1)
        acc ^= bit * cols[i]
    return acc


def _matmul(a, b):
    """GF(2) product a . b of matrices given as 32 uint32 columns."""
    return _apply(a, b)


def _matpow(cols, e):
    r = (np.uint32(1) << np.arange(32, dtype=np.uint32)).astype(np.uint32)  # identity
    base = cols.copy()
    while e:
        if e & 1:
            r = _matmul(base, r)
        base = _matmul(base, base)
        e >>= 1
    return r


def _stream_lanes(s0, n, L=4096, B=256):
    """Stream outputs 0 .. n-1 computed on J = ceil(n / L) lanes at once:
    lane j starts from the state after j L steps (GF(2) jumps, two levels:
    blocks of B lanes apart sequentially, lanes within a block vectorized)."""
    one = _powers()[0]                    # columns of one step
    jl = _matpow(one, L)                  # L steps
    jlb = _matpow(one, L * B)             # L B steps
    J = -(-n // L)
    nb = -(-J // B)
    heads = np.empty(nb, np.uint32)
    h = np.uint32(s0)
    for b in range(nb):
        heads[b] = h
        h = _apply(jlb, h)
    starts = np.empty((nb, B), np.uint32)
    starts[:, 0] = heads
    for k in range(1, B):
        starts[:, k] = _apply(jl, starts[:, k - 1])
    x = starts.ravel()[:J].copy()
    out = np.empty((J, L), np.uint32)
    for t in range(L):
        x = _step(x)
        out[:, t] = x
    return out.ravel()[:n]


def xorshift_stream(seed, n):
    """The first n outputs of xorshift32 from `seed` (0 -> 0x9e3779b9)."""
    s = np.uint32(seed if seed else 0x9E3779B9)
    if n > (1 << 24):
        return _stream_lanes(s, n)
    cols = _powers()
    out = np.empty(n, np.uint32)
    done = 0
    while done < n:
        take = min(_BLOCK, n - done)
        acc = np.zeros(take, np.uint32)
        for i in range(32):
            if (int(s) >> i) & 1:
                acc ^= cols[:take, i]
        out[done:done + take] = acc
        s = np.uint32(acc[-1]) if take == _BLOCK else s
        done += take
    return out


def rand(seed, scale, n):
    x = xorshift_stream(seed, n)
    u = (x >> np.uint32(8)).astype(np.float32) / np.float32(16777216.0)
    return ((np.float32(2.0) * u - np.float32(1.0)) * np.float32(scale)).astype(np.float32)


def normal(seed, sigma, n):
    """N(0, sigma) by Box-Muller over consecutive xorshift32 pairs (in f64,
    rounded once to f32); processed in chunks so that large n stays within
    about 3 x (4 n) bytes of memory."""
    m = (n + 1) // 2
    x = xorshift_stream(seed, 2 * m)
    out = np.empty(2 * m, np.float32)
    step = 1 << 24
    for i in range(0, m, step):
        j = min(m, i + step)
        u1 = ((x[2 * i:2 * j:2] >> np.uint32(8)).astype(np.float64) + 1.0) / 16777216.0
        u2 = (x[2 * i + 1:2 * j:2] >> np.uint32(8)).astype(np.float64) / 16777216.0
        r = np.sqrt(-2.0 * np.log(u1))
        out[2 * i:2 * j:2] = (r * np.cos(2.0 * np.pi * u2) * sigma).astype(np.float32)
        out[2 * i + 1:2 * j:2] = (r * np.sin(2.0 * np.pi * u2) * sigma).astype(np.float32)
    return out[:n]


def bits01(seed, n):
    """Uniform {0, 1} entries: the top bit of each xorshift32 output."""
    return (xorshift_stream(seed, n) >> np.uint32(31)).astype(np.float32)


def quantize_rtn(w, bits, axis):
    """w: f32 param (rank 2). Returns (codes int8 in the param's own layout,
    scales f32 per channel) as `tgc quantize --method rtn` writes them."""
    lim = 127 if bits == 8 else 7
    W = np.asarray(w, np.float64)
    if axis == 1:
        W = W.T  # channels are columns
    C, K = W.shape
    amax = np.abs(W).max(axis=1)
    best = np.full(C, np.inf)
    bs = np.where(amax == 0, 1e-8, amax / lim)
    for g in range(10):
        s = amax * (1.0 - 0.05 * g) / lim
        with np.errstate(divide="ignore", invalid="ignore"):
            code = np.clip(np.rint(W / s[:, None]), -lim, lim)
        code = np.where(s[:, None] > 0, code, 0.0)
        d = W - s[:, None] * code
        e = np.cumsum(d * d, axis=1)[:, -1]  # summed in index order, as the reference does
        better = (e < best) & (amax > 0)
        best = np.where(better, e, best)
        bs = np.where(better, s, bs)
    with np.errstate(divide="ignore", invalid="ignore"):
        codes = np.clip(np.rint(W / bs[:, None]), -lim, lim)
    codes = np.where(bs[:, None] > 0, codes, 0.0).astype(np.int8)
    if axis == 1:
        codes = codes.T
    return np.ascontiguousarray(codes), bs.astype(np.float32)


# ---- TGIR text ----

def _num_block(vals, fmt="%.9g", per_line=8, pad="\n         "):
    """Numbers the way the reference's ir_write lays them out (src/ir.c:166,
    :174-177): each as ' %.9g', a line break before every per_line-th."""
    out = []
    for i, v in enumerate(np.asarray(vals).ravel()):
        if i and i % per_line == 0:
            out.append(pad)
        out.append(" " + fmt % v)
    return "".join(out)


def _codes_text(codes):
    """Codes as fixed-width tokens, 24 per line (any spacing is valid TGIR):
    3 characters for int4 codes, 5 for int8."""
    c = np.asarray(codes, np.int64).ravel()
    w = 3 if c.size == 0 or np.abs(c).max() <= 7 else 5
    dt = "S%d" % w
    table = np.array([("%*d" % (w, v)).encode() for v in range(-127, 128)], dtype=dt)
    toks = table[c + 127]
    n = toks.size
    pad = (-n) % 24
    if pad:
        toks = np.concatenate([toks, np.array([b""] * pad, dtype=dt)])
    lines = toks.reshape(-1, 24)
    body = b"\n            ".join(b"".join(row) for row in lines)
    return body.decode()


def param_f32(name, arr):
    arr = np.asarray(arr, np.float32)
    shape = " ".join(str(d) for d in arr.shape)
    return "  (param %s (f32 %s)\n    (data%s))\n" % (name, shape, _num_block(arr.ravel()))


def param_quant(name, codes, scales, bits, axis):
    shape = " ".join(str(d) for d in codes.shape)
    sc = _num_block(scales, per_line=8, pad="\n            ")
    return "  (param %s (f32 %s)\n    (quant %d %d\n      (scale%s)\n      (codes %s)))\n" % (
        name, shape, bits, axis, sc, _codes_text(codes))


def mlp3_tgir(name, weights, bits):
    """rmsnorm(W3 @ tanh(W2 @ tanh(W1 @ x))) with int-`bits` W (axis 0)."""
    W1, W2, W3 = weights
    out = ["(tgir 1\n  (model %s)\n" % name]
    for nm, w in (("W1", W1), ("W2", W2), ("W3", W3)):
        if bits:
            c, s = quantize_rtn(w, bits, 0)
            out.append(param_quant(nm, c, s, bits, 0))
        else:
            out.append(param_f32(nm, w))
    d_in, h1, h2, d_out = W1.shape[1], W1.shape[0], W2.shape[0], W3.shape[0]
    out.append("  (input x (f32 %d))\n  (block\n" % d_in)
    out.append("    (%%0 (f32 %d) (matmul W1 x))\n    (%%1 (f32 %d) (tanh %%0))\n" % (h1, h1))
    out.append("    (%%2 (f32 %d) (matmul W2 %%1))\n    (%%3 (f32 %d) (tanh %%2))\n" % (h2, h2))
    out.append("    (%%4 (f32 %d) (matmul W3 %%3))\n    (%%5 (f32 %d) (rmsnorm %%4))\n" % (d_out, d_out))
    out.append("  )\n  (output %5))\n")
    return "".join(out)


def linear_tgir(name, W, bits):
    """W @ x with W quantized per output channel (axis 0)."""
    c, s = quantize_rtn(W, bits, 0)
    C, K = W.shape
    return "".join([
        "(tgir 1\n  (model %s)\n" % name, param_quant("W", c, s, bits, 0),
        "  (input x (f32 %d))\n  (block\n    (%%0 (f32 %d) (matmul W x))\n  )\n  (output %%0))\n" % (K, C),
    ])


def linear_tgir_codes(name, codes, scales, bits, axis=1):
    """One quantized product with the given codes (int8 values, the param's
    own layout) and per-channel scales: x @ W for axis 1 (W [K][C]), W @ x
    for axis 0 (W [C][K])."""
    codes = np.asarray(codes, np.int8)
    if axis == 1:
        K, C = codes.shape
        body = "  (input x (f32 %d))\n  (block\n    (%%0 (f32 %d) (matmul x W))\n  )\n  (output %%0))\n" % (K, C)
    else:
        C, K = codes.shape
        body = "  (input x (f32 %d))\n  (block\n    (%%0 (f32 %d) (matmul W x))\n  )\n  (output %%0))\n" % (K, C)
    return "(tgir 1\n  (model %s)\n" % name + param_quant("W", codes, scales, bits, axis) + body


# ---- BASELINE.json configurations ----

def config1(rows=65536):
    """Config 1: 512 -> 2048 -> 2048 -> 512 MLP, tanh, rmsnorm, --bits 8, weights
    rand(1, 0.05) (each param restarts the seed-1 stream, as three
    `rand(1, 0.05)` initializers would), inputs N(0, 1) seed 0."""
    W1 = rand(1, 0.05, 2048 * 512).reshape(2048, 512)
    W2 = rand(1, 0.05, 2048 * 2048).reshape(2048, 2048)
    W3 = rand(1, 0.05, 512 * 2048).reshape(512, 2048)
    x = normal(0, 1.0, rows * 512).reshape(rows, 512)
    return mlp3_tgir("mlp3", (W1, W2, W3), 8), x


def config2_weight():
    """Config 2: W 4096 x 4096 ~ N(0, 0.02) (seed 102: BASELINE gives no weight
    seed), int4 per output channel."""
    return normal(102, 0.02, 4096 * 4096).reshape(4096, 4096)


def config2(rows=4096):
    W = config2_weight()
    x = normal(2, 1.0, rows * 4096).reshape(rows, 4096)
    return linear_tgir("linear4096", W, 4), x


def latent_reasoner_tgir():
    """Config 4's model: examples/latent_reasoner's architecture with rand
    seeds 11/23/37/41 and b_core = fill(0.01), in the instruction order the
    reference lowers it to."""
    w_emb = rand(11, 0.35, 128).reshape(16, 8)
    w_core = rand(23, 0.12, 256).reshape(16, 16)
    w_inj = rand(37, 0.10, 256).reshape(16, 16)
    w_out = rand(41, 0.5, 64).reshape(4, 16)
    parts = ["(tgir 1\n  (model latent_reasoner)\n"]
    for nm, v in (("w_emb", w_emb), ("b_emb", np.zeros(16, np.float32)), ("w_core", w_core), ("w_inj", w_inj),
                  ("b_core", np.full(16, 0.01, np.float32)), ("w_out", w_out), ("b_out", np.zeros(4, np.float32))):
        parts.append(param_f32(nm, v))
    parts.append("""  (input x (f32 8))
  (block
    (%8 (f32 16) (matmul w_emb x))
    (%9 (f32 16) (add %8 b_emb))
    (%10 (f32 16) (rmsnorm %9))
    (%11 (f32 16) (think %10 32 9.99999975e-05
      (%12 (f32 16) (matmul w_core %11))
      (%13 (f32 16) (matmul w_inj %10))
      (%14 (f32 16) (add %12 %13))
      (%15 (f32 16) (add %14 b_core))
      (%16 (f32 16) (tanh %15))
      (yield %16)))
    (%17 (f32 4) (matmul w_out %11))
    (%18 (f32 4) (add %17 b_out))
    (%19 (f32 4) (softmax %18))
  )
  (output %19))
""")
    return "".join(parts)


def config4_rows(rows=1048576):
    return bits01(4, rows * 8).reshape(rows, 8)


def ssm_tgir(name="ssm", d_model=256, d_inner=512, n_state=16, dt_rank=16, T=512, blocks=4, classes=8, bits=8,
             seed=105):
    """Config 5's model: a Mamba-1-style selective-SSM sequence classifier.

    The reference has no builtin SSM block; this is the block (one sequence
    of T steps, rows of the tensors are time steps):
        xi = x @ Wx, z = x @ Wz                      (d_model -> d_inner each)
        u  = silu(xi)
        dt = softplus((u @ Wdtin) @ Wdt + bdt)       (d_inner -> dt_rank -> d_inner)
        B  = u @ WB, C = u @ WC                      (d_inner -> n_state)
        scan over t, carry h[d_inner, n_state] = 0:
            h   = exp(dt_t[:, None] * A) * h + outer(dt_t * u_t, B_t)
            y_t = h @ C_t
        y  = (y + u * D) * silu(z)
        x' = rmsnorm(x + y @ Wo)                     (d_inner -> d_model)
    and the head: p = mean over t of x (pool @ x, pool the 1/T vector),
    softmax(p @ Whead). A = -(1 .. n_state) per channel (A_log = log n), D = 1,
    bdt = softplus^-1(0.01). Every matmul weight is N(0, 0.02), drawn in
    order from one normal(seed) stream, and quantized per output channel on
    axis 1 (x @ W, as tgc quantize writes x @ W params)."""
    shapes = []
    for b in range(blocks):
        shapes += [("Wx%d" % b, (d_model, d_inner)), ("Wz%d" % b, (d_model, d_inner)),
                   ("Wdtin%d" % b, (d_inner, dt_rank)), ("Wdt%d" % b, (dt_rank, d_inner)),
                   ("WB%d" % b, (d_inner, n_state)), ("WC%d" % b, (d_inner, n_state)), ("Wo%d" % b, (d_inner, d_model))]
    shapes.append(("Whead", (d_model, classes)))
    total = sum(r * c for _, (r, c) in shapes)
    stream = normal(seed, 0.02, total)
    parts = ["(tgir 1\n  (model %s)\n" % name]
    off = 0
    for nm, (r, c) in shapes:
        w = stream[off:off + r * c].reshape(r, c)
        off += r * c
        if bits:
            codes, sc = quantize_rtn(w, bits, 1)
            parts.append(param_quant(nm, codes, sc, bits, 1))
        else:
            parts.append(param_f32(nm, w))
    A = -np.tile(np.arange(1, n_state + 1, dtype=np.float32), (d_inner, 1))
    parts.append(param_f32("A", A))
    parts.append(param_f32("D", np.ones(d_inner, np.float32)))
    parts.append(param_f32("bdt", np.full(d_inner, np.log(np.expm1(0.01)), np.float32)))
    parts.append(param_f32("h0", np.zeros((d_inner, n_state), np.float32)))
    parts.append(param_f32("pool", np.full(T, 1.0 / T, np.float32)))
    parts.append("  (input x (f32 %d %d))\n  (block\n" % (T, d_model))
    v = [0]

    def new():
        v[0] += 1
        return "%%%d" % v[0]

    lines = []

    def op(shape, expr):
        r = new()
        lines.append("    (%s (f32 %s) %s)\n" % (r, " ".join(str(d) for d in shape), expr))
        return r

    x = "x"
    for b in range(blocks):
        xi = op((T, d_inner), "(matmul %s Wx%d)" % (x, b))
        z = op((T, d_inner), "(matmul %s Wz%d)" % (x, b))
        u = op((T, d_inner), "(silu %s)" % xi)
        dtl = op((T, dt_rank), "(matmul %s Wdtin%d)" % (u, b))
        Bm = op((T, n_state), "(matmul %s WB%d)" % (u, b))
        Cm = op((T, n_state), "(matmul %s WC%d)" % (u, b))
        dtp = op((T, d_inner), "(matmul %s Wdt%d)" % (dtl, b))
        dta = op((T, d_inner), "(add %s bdt)" % dtp)
        dt = op((T, d_inner), "(softplus %s)" % dta)
        du = op((T, d_inner), "(mul %s %s)" % (dt, u))
        h, dtt, dut, bt, ct = new(), new(), new(), new(), new()
        dtc, da0, da, ha, dbu, hn, yt, ys = (new() for _ in range(8))
        lines.append("    (scan %d forward\n" % T)
        lines.append("      (carry %s (f32 %d %d) h0)\n" % (h, d_inner, n_state))
        lines.append("      (in %s (f32 %d) %s)\n      (in %s (f32 %d) %s)\n" % (dtt, d_inner, dt, dut, d_inner, du))
        lines.append("      (in %s (f32 %d) %s)\n      (in %s (f32 %d) %s)\n" % (bt, n_state, Bm, ct, n_state, Cm))
        lines.append("      (body\n")
        lines.append("        (%s (f32 %d 1) (reshape %s))\n" % (dtc, d_inner, dtt))
        lines.append("        (%s (f32 %d %d) (mul %s A))\n" % (da0, d_inner, n_state, dtc))
        lines.append("        (%s (f32 %d %d) (exp %s))\n" % (da, d_inner, n_state, da0))
        lines.append("        (%s (f32 %d %d) (mul %s %s))\n" % (ha, d_inner, n_state, da, h))
        lines.append("        (%s (f32 %d %d) (outer %s %s))\n" % (dbu, d_inner, n_state, dut, bt))
        lines.append("        (%s (f32 %d %d) (add %s %s))\n" % (hn, d_inner, n_state, ha, dbu))
        lines.append("        (%s (f32 %d) (matmul %s %s))\n" % (yt, d_inner, hn, ct))
        lines.append("      )\n      (next %s %s)\n      (emit %s (f32 %d %d) %s)\n    )\n" % (h, hn, ys, T, d_inner, yt))
        yd = op((T, d_inner), "(mul %s D)" % u)
        y1 = op((T, d_inner), "(add %s %s)" % (ys, yd))
        sz = op((T, d_inner), "(silu %s)" % z)
        y2 = op((T, d_inner), "(mul %s %s)" % (y1, sz))
        o = op((T, d_model), "(matmul %s Wo%d)" % (y2, b))
        r = op((T, d_model), "(add %s %s)" % (x, o))
        x = op((T, d_model), "(rmsnorm %s)" % r)
    p = op((d_model,), "(matmul pool %s)" % x)
    lg = op((classes,), "(matmul %s Whead)" % p)
    out = op((classes,), "(softmax %s)" % lg)
    parts.extend(lines)
    parts.append("  )\n  (output %s))\n" % out)
    return "".join(parts)


def qwen3_weights(L, D, NQ, NKV, HD, FF, V, seed=3, sigma=0.02):
    """Random-init weights of a Qwen3-shaped decoder, drawn in order from one
    normal(seed, sigma) stream: E [V, D], then per layer Wq_h (D, HD) for the
    NQ query heads, Wk_j and Wv_j (D, HD) for the NKV KV heads, Wo_h (HD, D),
    Wg and Wu (D, FF), Wd (FF, D). RMSNorm gains are 1 (the usual init) and
    the LM head is E transposed (tied embeddings, examples/qwen3/import.py:49)."""
    shapes = [("E", (V, D))]
    for l in range(L):
        shapes += [("Wq_%d_%d" % (l, h), (D, HD)) for h in range(NQ)]
        shapes += [("Wk_%d_%d" % (l, j), (D, HD)) for j in range(NKV)]
        shapes += [("Wv_%d_%d" % (l, j), (D, HD)) for j in range(NKV)]
        shapes += [("Wo_%d_%d" % (l, h), (HD, D)) for h in range(NQ)]
        shapes += [("Wg_%d" % l, (D, FF)), ("Wu_%d" % l, (D, FF)), ("Wd_%d" % l, (FF, D))]
    total = sum(r * c for _, (r, c) in shapes)
    stream = normal(seed, sigma, total)
    w, off = {}, 0
    for nm, (r, c) in shapes:
        w[nm] = stream[off:off + r * c].reshape(r, c)
        off += r * c
    return w


def rope_tables(T, HD, theta=1e6):
    """cos/sin [T, HD] (rotate-half convention) and the [HD, HD] matrix with
    x @ Rot = rotate_half(x), as examples/qwen3/import.py:80-89 builds them."""
    inv = theta ** (-(np.arange(0, HD, 2) / HD))
    ang = np.outer(np.arange(T), inv)
    cos = np.concatenate([np.cos(ang), np.cos(ang)], axis=1).astype(np.float32)
    sin = np.concatenate([np.sin(ang), np.sin(ang)], axis=1).astype(np.float32)
    rot = np.zeros((HD, HD), np.float32)
    for i in range(HD // 2):
        rot[i + HD // 2, i] = -1.0
        rot[i, i + HD // 2] = 1.0
    return cos, sin, rot


def qwen3_tgir(name="qwen3", L=28, D=1024, NQ=16, NKV=8, HD=128, FF=3072, V=151936, T=512, bits=4, seed=3, files=None,
               quantizer=None, rope_len=None, cache=None):
    """Config 3's model at fixed sequence length T: the graph
    examples/qwen3/import.py:110-130 emits (per-head rank-2 matmuls, GQA with
    NQ / NKV query heads per KV head, rotate-half RoPE as x * cos + (x @ Rot)
    * sin, causal mask added before softmax, SwiGLU MLP, tied LM head, output
    the logits of the last position), lowered to TGIR. One row is one
    sequence: f32[T] token ids. Every param `tgc quantize --bits 4` would
    quantize (rank-2 matmul operands: all linear weights, the LM head and Rot)
    is quantized RTN int`bits` on axis 1 (x @ W); E, the RoPE tables and the
    mask stay f32.

    files: a directory; the params are then written there as raw arrays and
    the text refers to them with the backend's data-file / scale-file /
    codes-file forms (a full-size model as TGIR text would be several GB).
    quantizer: an RTN function with quantize_rtn's signature (the library's
    native one for full size); quantize_rtn by default.
    rope_len: also emit the RoPE tables `rope_cos` / `rope_sin` with that many
    rows (the KV-cache decoder reads them for positions beyond T; the
    fixed-length graph does not use them). Row p equals row p of cosT / sinT.
    cache: a dict kept by the caller across calls with the same files
    directory, weights and bits: the params that do not depend on T are
    written once and their text reused (models of several lengths T share
    one set of weight files)."""
    if cache is not None and files is None:
        raise ValueError("cache needs a files directory")
    key = (L, D, NQ, NKV, HD, FF, V, bits, seed)
    if cache is not None and cache.get("key", key) != key:
        raise ValueError("cache holds another model's weights")
    w = qwen3_weights(L, D, NQ, NKV, HD, FF, V, seed) if cache is None or "E" not in cache else None
    cos, sin, rot = rope_tables(T, HD)
    mask = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], 0.0, -1e9).astype(np.float32)
    ones_d, ones_hd = np.ones(D, np.float32), np.ones(HD, np.float32)
    parts = ["(tgir 1\n  (model %s)\n" % name]
    rtn = quantizer or quantize_rtn

    def f32p(nm, arr, by_t=False):
        if files is None:
            return param_f32(nm, arr() if callable(arr) else arr)
        if cache is not None and not by_t and nm in cache:
            return cache[nm]
        arr = np.ascontiguousarray(arr() if callable(arr) else arr, np.float32)
        path = os.path.join(files, nm + (".T%d" % T if by_t else "") + ".f32")
        arr.tofile(path)
        text = "  (param %s (f32 %s)\n    (data-file %s))\n" % (nm, " ".join(str(d) for d in arr.shape), path)
        if cache is not None and not by_t:
            cache[nm] = text
            cache["key"] = key
        return text

    def quant(nm, arr):
        if cache is not None and nm in cache:
            parts.append(cache[nm])
            return
        codes, sc = rtn(arr() if callable(arr) else arr, bits, 1)
        if files is None:
            parts.append(param_quant(nm, codes, sc, bits, 1))
            return
        cpath, spath = os.path.join(files, nm + ".codes"), os.path.join(files, nm + ".scale")
        np.ascontiguousarray(codes, np.int8).tofile(cpath)
        np.ascontiguousarray(sc, np.float32).tofile(spath)
        text = "  (param %s (f32 %s)\n    (quant %d 1 (scale-file %s) (codes-file %s)))\n" % (
            nm, " ".join(str(d) for d in codes.shape), bits, spath, cpath)
        if cache is not None:
            cache[nm] = text
            cache["key"] = key
        parts.append(text)

    parts.append(f32p("E", lambda: w["E"]))
    quant("LM", lambda: np.ascontiguousarray(w["E"].T))
    parts.append(f32p("lnf", ones_d))
    parts.append(f32p("cosT", cos, by_t=True))
    parts.append(f32p("sinT", sin, by_t=True))
    quant("Rot", rot)
    parts.append(f32p("mask", mask, by_t=True))
    if rope_len:
        rc, rs, _ = rope_tables(rope_len, HD)
        parts.append(f32p("rope_cos", rc, by_t=True))
        parts.append(f32p("rope_sin", rs, by_t=True))
    parts.append(f32p("lastidx", np.array([T - 1], np.float32), by_t=True))
    for l in range(L):
        for nm in ("ln1_%d", "ln2_%d"):
            parts.append(f32p(nm % l, ones_d))
        for nm in ("qn_%d", "kn_%d"):
            parts.append(f32p(nm % l, ones_hd))
        for h in range(NQ):
            quant("Wq_%d_%d" % (l, h), lambda k="Wq_%d_%d" % (l, h): w[k])
            quant("Wo_%d_%d" % (l, h), lambda k="Wo_%d_%d" % (l, h): w[k])
        for j in range(NKV):
            quant("Wk_%d_%d" % (l, j), lambda k="Wk_%d_%d" % (l, j): w[k])
            quant("Wv_%d_%d" % (l, j), lambda k="Wv_%d_%d" % (l, j): w[k])
        for nm in ("Wg_%d", "Wu_%d", "Wd_%d"):
            quant(nm % l, lambda k=nm % l: w[k])
    parts.append("  (input ids (f32 %d))\n  (block\n" % T)
    v = [0]
    lines = []

    def op(shape, expr):
        v[0] += 1
        r = "%%%d" % v[0]
        lines.append("    (%s (f32%s) %s)\n" % (r, "".join(" %d" % d for d in shape), expr))
        return r

    def rotary(x):  # x * cosT + (x @ Rot) * sinT
        a = op((T, HD), "(mul %s cosT)" % x)
        b = op((T, HD), "(matmul %s Rot)" % x)
        c = op((T, HD), "(mul %s sinT)" % b)
        return op((T, HD), "(add %s %s)" % (a, c))

    scale = op((), "(const %.9g)" % (1.0 / np.sqrt(HD)))
    h = op((T, D), "(take E ids)")
    for l in range(L):
        n = op((T, D), "(mul %s ln1_%d)" % (op((T, D), "(rmsnorm %s)" % h), l))
        ks, vs = [], []
        for j in range(NKV):
            a = op((T, HD), "(matmul %s Wk_%d_%d)" % (n, l, j))
            ks.append(rotary(op((T, HD), "(mul %s kn_%d)" % (op((T, HD), "(rmsnorm %s)" % a), l))))
            vs.append(op((T, HD), "(matmul %s Wv_%d_%d)" % (n, l, j)))
        terms = []
        for hh in range(NQ):
            j = hh // (NQ // NKV)
            a = op((T, HD), "(matmul %s Wq_%d_%d)" % (n, l, hh))
            q = rotary(op((T, HD), "(mul %s qn_%d)" % (op((T, HD), "(rmsnorm %s)" % a), l)))
            kt = op((HD, T), "(transpose %s)" % ks[j])
            sc = op((T, T), "(mul %s %s)" % (op((T, T), "(matmul %s %s)" % (q, kt)), scale))
            s = op((T, T), "(softmax %s)" % op((T, T), "(add %s mask)" % sc))
            terms.append(op((T, D), "(matmul %s Wo_%d_%d)" % (op((T, HD), "(matmul %s %s)" % (s, vs[j])), l, hh)))
        acc = terms[0]
        for t_ in terms[1:]:
            acc = op((T, D), "(add %s %s)" % (acc, t_))
        h = op((T, D), "(add %s %s)" % (h, acc))
        n = op((T, D), "(mul %s ln2_%d)" % (op((T, D), "(rmsnorm %s)" % h), l))
        g = op((T, FF), "(silu %s)" % op((T, FF), "(matmul %s Wg_%d)" % (n, l)))
        u = op((T, FF), "(matmul %s Wu_%d)" % (n, l))
        h = op((T, D), "(add %s %s)" % (h, op((T, D), "(matmul %s Wd_%d)" % (op((T, FF), "(mul %s %s)" % (g, u)), l))))
    nf = op((T, D), "(mul %s lnf)" % op((T, D), "(rmsnorm %s)" % h))
    logits = op((T, V), "(matmul %s LM)" % nf)
    out = op((V,), "(reshape %s)" % op((1, V), "(take %s lastidx)" % logits))
    parts.extend(lines)
    parts.append("  )\n  (output %s))\n" % out)
    return "".join(parts)


def config3_prompts(seqs=64, T=512, V=151936, seed=3):
    """Config 3 prompts: seqs rows of T token ids uniform in [0, V), as f32
    (exact below 2^24), from xorshift32(seed): id = x mod V."""
    x = xorshift_stream(seed, seqs * T)
    return (x % np.uint32(V)).astype(np.float32).reshape(seqs, T)


def config5_rows(rows=4096, T=512, d_model=256, seed=5):
    """Config 5 inputs: rows sequences of T steps of f32[d_model] ~ N(0, 1)."""
    return normal(seed, 1.0, rows * T * d_model).reshape(rows, T * d_model)
