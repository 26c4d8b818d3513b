"""Seeded input cases shared by the golden-fixture writer, the oracle tests and the GPU
parity tests. Every case is a dict of numpy arrays and scalars; nothing here computes
an expected value.
"""

from __future__ import annotations

import numpy as np

from oracle_ctypes import fill_lcg, lcg_int8


def _rng(seed):
    return np.random.default_rng(seed)


def quant_cases():
    """accel::MatMulQuantized inputs (src/sim_device.cc:541-602)."""
    cases = []
    # tests/test_runtime.cc:325-392: per-row (axis 0) scale + zero, then a scalar scale.
    m, k, n = 8, 160, 300
    a, seed = fill_lcg(m * k, 3)
    q, _ = lcg_int8(k * n, seed)
    rows = np.arange(k)
    scale = ((rows % 5).astype(np.float32) * np.float32(0.25) + np.float32(0.5)).astype(np.float32)
    zero = (rows % 7 - 3).astype(np.int8)
    spec = dict(q=q, scale=scale, zero=zero, shape=[k, n], axis=0, offset=0)
    cases.append(dict(name="row_scale_zero", m=m, k=k, n=n, a=a.reshape(m, k), bq=spec))
    cases.append(dict(name="scalar_scale", m=m, k=k, n=n, a=a.reshape(m, k),
                      bq=dict(q=q, scale=np.array([0.5], np.float32), zero=None, shape=[k, n], axis=-1, offset=0)))
    # The DQ KAT of tests/test_ep.py:336-343 (want[0, 0] = -48.5).
    cases.append(dict(name="dq_kat", m=2, k=2, n=2, a=np.array([[1, 2], [0, -1]], np.float32),
                      bq=dict(q=np.array([-128, 127, 1, -2], np.int8), scale=np.array([0.5, 2.0], np.float32),
                              zero=np.array([1, -3], np.int8), shape=[2, 2], axis=0, offset=0)))
    # Per-output-column scale (axis 1), zero point, the C1/C3 layout at small size.
    r = _rng(11)
    for (m, k, n, with_zero) in [(1, 64, 96, False), (4, 96, 160, True), (16, 128, 72, False), (37, 70, 130, True)]:
        q = r.integers(-127, 128, size=k * n, dtype=np.int8)
        scale = r.uniform(1e-3, 1e-2, size=n).astype(np.float32)
        zero = r.integers(-4, 5, size=n, dtype=np.int8) if with_zero else None
        a = r.standard_normal((m, k)).astype(np.float32)
        cases.append(dict(name=f"col_{m}x{k}x{n}", m=m, k=k, n=n, a=a,
                          bq=dict(q=q, scale=scale, zero=zero, shape=[k, n], axis=1, offset=0)))
    # Rank-3 weight [2, k, n] with the scale on the batch axis (axis 0), second batch (offset k*n).
    m, k, n = 3, 24, 40
    q = r.integers(-127, 128, size=2 * k * n, dtype=np.int8)
    scale = np.array([0.25, 0.0078125], np.float32)
    zero = np.array([2, -1], np.int8)
    a = r.standard_normal((m, k)).astype(np.float32)
    cases.append(dict(name="batch_axis", m=m, k=k, n=n, a=a,
                      bq=dict(q=q, scale=scale, zero=zero, shape=[2, k, n], axis=0, offset=k * n)))
    # Rank-3 weight, per-column scale, second batch.
    scale = r.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    cases.append(dict(name="batch_col", m=m, k=k, n=n, a=a,
                      bq=dict(q=q, scale=scale, zero=None, shape=[2, k, n], axis=2, offset=k * n)))
    # Quantized left operand (A-side plane), per-row scale on A's rows.
    m, k, n = 5, 33, 21
    qa = r.integers(-127, 128, size=m * k, dtype=np.int8)
    sa = r.uniform(0.01, 0.1, size=m).astype(np.float32)
    b = r.standard_normal((k, n)).astype(np.float32)
    cases.append(dict(name="a_side", m=m, k=k, n=n, b=b,
                      aq=dict(q=qa, scale=sa, zero=None, shape=[m, k], axis=0, offset=0)))
    # k = 0 overwrites C with zeros.
    cases.append(dict(name="k_zero", m=3, k=0, n=4, a=np.zeros((3, 0), np.float32),
                      bq=dict(q=np.zeros(1, np.int8), scale=np.array([1.0], np.float32), zero=None, shape=[0, 4],
                              axis=-1, offset=0)))
    return cases


def epilogue_cases():
    """SimDevice::GemmEpilogue inputs (src/sim_device.cc:211-245)."""
    r = _rng(21)
    m, n = 7, 33
    base = r.standard_normal((m, n)).astype(np.float32) * np.float32(3)
    base[0, 0] = np.inf
    base[0, 1] = -np.inf
    base[0, 2] = np.nan
    base[0, 3] = -0.0
    base[0, 4] = 0.0
    cases = []
    shapes = {"none": None, "row": [n], "col": [m, 1], "bcast_row": [1, n], "full": [m, n], "scalar1": [1],
              "rank0": []}
    for act in (0, 1, 2):
        for bname, bshape in shapes.items():
            if bshape is None:
                bias = None
                bshape = []
            else:
                count = int(np.prod(bshape)) if bshape else 1
                bias = r.standard_normal(count).astype(np.float32)
            for (alpha, beta) in [(1.0, 1.0), (-1.5, 0.75)]:
                cases.append(dict(name=f"a{act}_{bname}_{alpha}", c=base, alpha=alpha, beta=beta, bias=bias,
                                  bias_shape=bshape, act=act))
    return cases


def rmsnorm_cases():
    r = _rng(31)
    x = r.standard_normal((6, 576)).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(576)).astype(np.float32)
    return [dict(name="576", x=x, w=w, rows=4, dim=576, eps=1e-5, row_offset=2),
            dict(name="kat4", x=np.array([1, -1, 2, 0, 4, -2, 0.5, 3], np.float32),
                 w=np.array([1, 2, 0.5, 1.5], np.float32), rows=1, dim=4, eps=1e-5, row_offset=1)]


def embed_cases():
    r = _rng(41)
    table = r.standard_normal((50, 24)).astype(np.float32)
    return [dict(name="ok", ids=np.array([7, 3, 49, 0, 12], np.int32), id_offset=1, table=table, seq=4),
            dict(name="oov", ids=np.array([7, 50, 2], np.int32), id_offset=0, table=table, seq=3)]


def rope_cases():
    from oracle_ctypes import oracle

    r = _rng(51)
    cos, sin = oracle().rope_tables(16, 64, 100000.0)
    return [dict(name="q9", states=r.standard_normal((3, 9, 64)).astype(np.float32), cos=cos, sin=sin, seq=3,
                 heads=9, head_dim=64, position=5)]


def attention_cases():
    r = _rng(61)
    out = []
    for (seq, pos) in [(4, 3), (1, 11), (7, 0)]:
        total = seq + pos
        out.append(dict(name=f"s{seq}p{pos}", q=r.standard_normal((seq, 9, 64)).astype(np.float32),
                        k=r.standard_normal((total, 3, 64)).astype(np.float32),
                        v=r.standard_normal((total, 3, 64)).astype(np.float32), seq=seq, position=pos, heads=9,
                        kv_heads=3, head_dim=64))
    return out


def silu_add_cases():
    r = _rng(71)
    g = (r.standard_normal(1000) * 4).astype(np.float32)
    g[:4] = [0.0, -0.0, 80.0, -90.0]
    return [dict(name="1000", gate=g, up=r.standard_normal(1000).astype(np.float32))]


def sample_cases():
    """SimSampleToken inputs: the integer KATs of tests/test_sim_kernels.cc:187-231 plus seeded sweeps."""
    cases = [
        dict(logits=np.array([1, 3, 3], np.float32), temperature=0.0, rng=1, top_k=2),
        dict(logits=np.array([1, 3, 3], np.float32), temperature=-1.0, rng=1, top_k=0),
        dict(logits=np.array([1, 3, 0], np.float32), temperature=1.0, rng=1856, top_k=2),
        dict(logits=np.array([1, 3, 0], np.float32), temperature=1.0, rng=1856, top_k=0),
        dict(logits=np.array([1, 3, 0], np.float32), temperature=1.0, rng=0, top_k=0),
        dict(logits=np.zeros(65, np.float32), temperature=1.0, rng=1000, top_k=65),
        dict(logits=np.zeros(65, np.float32), temperature=1.0, rng=1000, top_k=64),
    ]
    r = _rng(81)
    for vocab in (50, 200, 1000):
        for t in (0.0, 0.7, 1.5):
            for top_k in (0, 1, 5, 64, 65, vocab, vocab + 3):
                for tie in (False, True):
                    logits = r.standard_normal(vocab).astype(np.float32) * np.float32(2)
                    if tie:
                        logits = np.round(logits).astype(np.float32)
                    cases.append(dict(logits=logits, temperature=t, rng=int(r.integers(1, 2**32 - 1)), top_k=top_k))
    return cases


def llama_config(name):
    if name == "tiny":
        return dict(vocab=256, hidden=64, layers=2, heads=4, kv_heads=2, intermediate=128, context=48, eps=1e-5,
                    rope_theta=100000.0)
    if name == "smol":  # SmolLM2-135M shape
        return dict(vocab=49152, hidden=576, layers=30, heads=9, kv_heads=3, intermediate=1536, context=640, eps=1e-5,
                    rope_theta=100000.0)
    if name == "smol3":  # SmolLM2-135M widths, 3 layers, short context
        return dict(vocab=49152, hidden=576, layers=3, heads=9, kv_heads=3, intermediate=1536, context=40, eps=1e-5,
                    rope_theta=100000.0)
    raise KeyError(name)


def llama_weights(config, seed, quantize=True):
    """Random-init Llama weights in Hugging Face layout ([out, in] matrices, [dim] norms).

    Linear weights (and the tied embedding / lm head) are N(0, 0.02), quantized per output
    row: s = max|w| / 127, q = rint(w / s); the float weight handed to the float reference is
    fl(q * s). Norm weights are N(1, 0.1). Returns (weights, quant) where weights is a list
    of (kind, layer, float array) and quant maps (kind, layer) -> (q int8 [out, in], s [out]).
    """
    r = _rng(seed)
    hid = config["hidden"]
    heads = config["heads"]
    kvh = config["kv_heads"]
    hd = hid // heads
    inter = config["intermediate"]
    vocab = config["vocab"]
    weights = []
    quant = {}

    def linear(kind, layer, rows, cols):
        w = (r.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        if quantize:
            s = (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32)
            s[s == 0] = np.float32(1)
            q = np.rint(w / s[:, None]).clip(-127, 127).astype(np.int8)
            w = (q.astype(np.float32) * s[:, None]).astype(np.float32)
            quant[(kind, layer)] = (q, s)
        weights.append((kind, layer, w))

    def norm(kind, layer):
        weights.append((kind, layer, (1 + 0.1 * r.standard_normal(hid)).astype(np.float32)))

    linear(1, -1, vocab, hid)  # embedding; the lm head is tied to it
    emb = weights[-1][2]
    weights.append((3, -1, emb))
    if quantize:
        quant[(3, -1)] = quant[(1, -1)]
    norm(2, -1)
    for layer in range(config["layers"]):
        norm(4, layer)
        norm(5, layer)
        linear(6, layer, heads * hd, hid)
        linear(7, layer, kvh * hd, hid)
        linear(8, layer, kvh * hd, hid)
        linear(9, layer, hid, heads * hd)
        linear(10, layer, inter, hid)
        linear(11, layer, inter, hid)
        linear(12, layer, hid, inter)
    return weights, quant


def llama_cases():
    cases = []
    cfg = llama_config("tiny")
    w, _ = llama_weights(cfg, 101)
    prompt = _rng(102).integers(0, cfg["vocab"], size=16).astype(np.int32)
    cases.append(dict(name="tiny_greedy", config=cfg, weights=w, weight_seed=101, prompt=prompt, max_new=24, eos=-1,
                      temperature=0.0, seed=0, top_k=0))
    cases.append(dict(name="tiny_topk", config=cfg, weights=w, weight_seed=101, prompt=prompt, max_new=24, eos=-1,
                      temperature=0.8, seed=7, top_k=12))
    cfg3 = llama_config("smol3")
    w3, _ = llama_weights(cfg3, 103)
    prompt3 = _rng(104).integers(0, cfg3["vocab"], size=20).astype(np.int32)
    cases.append(dict(name="smol3_greedy", config=cfg3, weights=w3, weight_seed=103, prompt=prompt3, max_new=12,
                      eos=-1, temperature=0.0, seed=0, top_k=0))
    return cases


def llama_full_case(sampled=False):
    """The SmolLM2-135M-shape forward: 30 layers, 512 prompt ids, 128 tokens, greedy (the
    configured workload) or top-k sampled (temperature 0.8, top 40, seed 11), whose ids do
    not settle on a fixed point."""
    cfg = llama_config("smol")
    w, q = llama_weights(cfg, 105)
    prompt = _rng(106).integers(0, cfg["vocab"], size=512).astype(np.int32)
    if sampled:
        return dict(name="smol_full_topk", config=cfg, weights=w, quant=q, prompt=prompt, max_new=128, eos=-1,
                    temperature=0.8, seed=11, top_k=40)
    return dict(name="smol_full_greedy", config=cfg, weights=w, quant=q, prompt=prompt, max_new=128, eos=-1,
                temperature=0.0, seed=0, top_k=0)


def complete_config():
    """The model of the completion cases: tiny widths, and the vocabulary of
    tests/golden/tokenizer_small.json (1220 tokens), so that every id decodes."""
    return dict(vocab=1220, hidden=64, layers=2, heads=4, kv_heads=2, intermediate=128, context=48, eps=1e-5,
                rope_theta=100000.0)


COMPLETE_WEIGHT_SEED = 107
