"""Writers of the reference's `.tmc` manifests for the importer tests.

The layout is the one the reference's exporters produce
(tools/export_decoder_llm.py:_write_archive, tools/export_kv_cache.py:
_write_archive): a text manifest plus a raw float32 payload named
`<manifest>.bin` beside it.  Reference results are computed here by the
oracle (decoder) or by a float64 numpy restatement of
workloads/pytorch/KVCache.py:MultiHeadAttentionKVCache (KV cache), not by
PyTorch.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

DECODER_KEYS = ("batch", "hidden_size", "heads", "intermediate_size", "vocabulary_size", "layers",
                "capacity", "prefill_length", "decode_count")
KV_KEYS = ("batch", "heads", "head_dimension", "capacity", "prefill_length", "decode_count")


def _payload(tensors: dict) -> tuple[np.ndarray, dict]:
    parts, ranges, offset = [], {}, 0
    for name, value in tensors.items():
        flat = np.asarray(value, np.float32).ravel()
        ranges[name] = (offset, flat.size)
        offset += flat.size
        parts.append(flat)
    return (np.concatenate(parts) if parts else np.zeros(0, np.float32)), ranges


def write_decoder_manifest(path, config: dict, tensors: dict, dtype=("F16", "F16"), version=2,
                           model_name="DecoderOnlyLLM", extra_lines=(), payload_name=None):
    """`dtype` = (requested, effective); version 1 writes one token, None
    omits the DTYPE line."""
    path = Path(path)
    payload, ranges = _payload(tensors)
    bin_name = payload_name or path.name + ".bin"
    payload.tofile(path.with_name(bin_name))
    lines = [f"TMC_DECODER_LLM {version}", f"MODEL {json.dumps(model_name)}",
             f"PAYLOAD {json.dumps(bin_name)}",
             "CONFIG " + " ".join(str(config[k]) for k in DECODER_KEYS) +
             f" {config['epsilon']:.9g}"]
    if dtype is not None:
        lines.append("DTYPE " + (dtype[0] if version == 1 else f"{dtype[0]} {dtype[1]}"))
    lines.append(f"TENSORS {len(ranges)}")
    lines += [f"TENSOR {json.dumps(n)} {o} {c}" for n, (o, c) in ranges.items()]
    lines.append("END")
    lines += list(extra_lines)
    path.write_text("\n".join(lines) + "\n")
    return path


def write_kv_manifest(path, config: dict, tensors: dict, steps: list, declared_steps=None,
                      step_indices=None):
    """steps: list of dicts with query, key, value, output, key_cache,
    value_cache (each an array)."""
    path = Path(path)
    fields = ("query", "key", "value", "output", "key_cache", "value_cache")
    named = dict(tensors)
    for i, step in enumerate(steps):
        for f in fields:
            named[f"__step{i}.{f}"] = step[f]
    payload, ranges = _payload(named)
    payload.tofile(path.with_name(path.name + ".bin"))
    plain = {n: r for n, r in ranges.items() if not n.startswith("__step")}
    lines = ["TMC_KV_CACHE 1", f"MODEL {json.dumps('MultiHeadAttentionKVCache')}",
             f"PAYLOAD {json.dumps(path.name + '.bin')}",
             "CONFIG " + " ".join(str(config[k]) for k in KV_KEYS),
             f"TENSORS {len(plain)}"]
    lines += [f"TENSOR {json.dumps(n)} {o} {c}" for n, (o, c) in plain.items()]
    lines.append(f"STEPS {len(steps) if declared_steps is None else declared_steps}")
    for i in range(len(steps)):
        index = i if step_indices is None else step_indices[i]
        spans = " ".join(f"{ranges[f'__step{i}.{f}'][0]} {ranges[f'__step{i}.{f}'][1]}"
                         for f in fields)
        lines.append(f"STEP {index} {spans}")
    lines.append("END")
    path.write_text("\n".join(lines) + "\n")
    return path


# ---------------------------------------------------------------- fixtures
def decoder_config(hidden=64, heads=4, layers=2, inter=128, vocab=128, capacity=32, prefill=8,
                   decode=8, epsilon=1e-5):
    """The reference exporter's defaults (export_decoder_llm.py:DEFAULT_CONFIG)."""
    return dict(batch=1, hidden_size=hidden, heads=heads, intermediate_size=inter,
                vocabulary_size=vocab, layers=layers, capacity=capacity, prefill_length=prefill,
                decode_count=decode, epsilon=epsilon)


def decoder_tensors(orc, config: dict, seed: int, page: int = 16):
    """fp16-representable weights (seeded), the interleaved RoPE tables and
    the oracle's prefill / decode references, named as the exporter names
    them.  The oracle runs the prefill as one decoder step whose rows are the
    prompt's tokens (the causal chunk rule) and then one step per token."""
    rng = np.random.default_rng(seed)
    H, I, V, L = (config["hidden_size"], config["intermediate_size"], config["vocabulary_size"],
                  config["layers"])
    NH, C, P = config["heads"], config["capacity"], config["prefill_length"]
    D = H // NH
    f16 = lambda a: orc.f16(np.asarray(a, np.float32))  # noqa: E731
    w = lambda *shape: f16(rng.standard_normal(shape) * 0.05)  # noqa: E731
    layers = [dict(input_norm=f16(rng.uniform(0.5, 1.5, H)), wq=w(H, H), wk=w(H, H), wv=w(H, H),
                   wo=w(H, H), post_norm=f16(rng.uniform(0.5, 1.5, H)), wg=w(I, H), wu=w(I, H),
                   wd=w(H, I)) for _ in range(L)]
    pos = np.arange(C, dtype=np.float64)[:, None]
    freq = 10000.0 ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    m = dict(embedding=f16(rng.standard_normal((V, H))), final_norm=f16(rng.uniform(0.5, 1.5, H)),
             lm_head=w(V, H), rope_cos=np.cos(pos * freq).astype(np.float32),
             rope_sin=np.sin(pos * freq).astype(np.float32), layers=layers)
    val = orc.f16_values
    tensors = {"embedding.weight": val(m["embedding"]), "final_norm.weight": val(m["final_norm"]),
               "lm_head.weight": val(m["lm_head"]), "rope.cosine": m["rope_cos"],
               "rope.sine": m["rope_sin"]}
    names = (("input_norm", "input_norm"), ("wq", "q"), ("wk", "k"), ("wv", "v"), ("wo", "o"),
             ("post_norm", "post_norm"), ("wg", "gate"), ("wu", "up"), ("wd", "down"))
    for l, lw in enumerate(layers):
        for key, name in names:
            tensors[f"layer{l}.{name}.weight"] = val(lw[key])
    cfg = dict(layers=L, hidden=H, heads=NH, head_dim=D, kv_heads=NH, intermediate=I,
               vocabulary=V, capacity=C, epsilon=config["epsilon"])
    max_pages = (C + page - 1) // page
    k = [np.zeros(max_pages * NH * page * D, np.uint16) for _ in range(L)]
    v = [np.zeros_like(x) for x in k]
    tables = np.tile(np.arange(max_pages, dtype=np.int32), (L, 1, 1))

    def caches(length):
        out_k, out_v = [], []
        for l in range(L):
            pk = k[l].reshape(max_pages, NH, page, D)
            pv = v[l].reshape(max_pages, NH, page, D)
            gather = lambda pool: np.stack(  # noqa: E731
                [pool[p // page, :, p % page, :] for p in range(length)], axis=1)
            out_k.append(val(gather(pk)))
            out_v.append(val(gather(pv)))
        return out_k, out_v

    prompt = rng.integers(0, V, P)
    t = np.tile(tables, (1, P, 1)).reshape(L, P, max_pages)
    logits, nxt = orc.decoder_step(m, cfg, k, v, page, max_pages, t, prompt, np.arange(1, P + 1))
    ck, cv = caches(P)
    steps = [("prefill", prompt, logits, nxt[-1:], ck, cv)]
    token = int(nxt[-1])
    for s in range(config["decode_count"]):
        lg, nx = orc.decoder_step(m, cfg, k, v, page, max_pages, tables, np.array([token]),
                                  np.array([P + s + 1]))
        ck, cv = caches(P + s + 1)
        steps.append((f"decode{s}", np.array([token]), lg, nx, ck, cv))
        token = int(nx[0])
    for prefix, toks, lg, nx, ck, cv in steps:
        tensors[f"{prefix}.tokens"] = toks
        tensors[f"{prefix}.logits"] = lg
        tensors[f"{prefix}.next_tokens"] = nx
        for l in range(L):
            tensors[f"{prefix}.layer{l}.key_cache"] = ck[l]
            tensors[f"{prefix}.layer{l}.value_cache"] = cv[l]
    return tensors


def oracle_decoder_run(orc, workload, prompt, decode_tokens, page: int = 16):
    """The oracle's decoder step (tmco_decoder_step) over an imported
    workload's weights, rounded to fp16 with the host rule as the gfx950
    decoder stores them: the prompt as one step whose rows are its tokens,
    then one step per given decode token.  Returns [(logits, next tokens,
    key caches, value caches)] per step, caches [heads, length, D] per
    layer."""
    plan = workload.plan
    L, NH = plan.layer_count, plan.attention.heads
    D, C = plan.attention.head_dimension, plan.attention.capacity
    H, I, V = NH * D, plan.intermediate_size, plan.vocabulary_size
    f16 = lambda a: orc.f16(np.asarray(a, np.float32))  # noqa: E731
    rows = lambda a, n: f16(np.asarray(a, np.float32).reshape(n, -1))  # noqa: E731
    layers = [dict(input_norm=f16(lw.input_norm_weight), wq=rows(lw.query_weight, H),
                   wk=rows(lw.key_weight, H), wv=rows(lw.value_weight, H),
                   wo=rows(lw.output_weight, H), post_norm=f16(lw.post_attention_norm_weight),
                   wg=rows(lw.gate_weight, I), wu=rows(lw.up_weight, I),
                   wd=rows(lw.down_weight, H)) for lw in workload.layers]
    m = dict(embedding=rows(workload.embedding_weight, V), final_norm=f16(workload.final_norm_weight),
             lm_head=rows(workload.language_model_head_weight, V),
             rope_cos=np.asarray(workload.rope_cosine, np.float32),
             rope_sin=np.asarray(workload.rope_sine, np.float32), layers=layers)
    cfg = dict(layers=L, hidden=H, heads=NH, head_dim=D, kv_heads=NH, intermediate=I,
               vocabulary=V, capacity=C, epsilon=plan.rms_norm_epsilon)
    max_pages = (C + page - 1) // page
    k = [np.zeros(max_pages * NH * page * D, np.uint16) for _ in range(L)]
    v = [np.zeros_like(x) for x in k]
    tables = np.tile(np.arange(max_pages, dtype=np.int32), (L, 1, 1))

    def caches(length):
        out = []
        for pools in (k, v):
            per_layer = []
            for l in range(L):
                pool = pools[l].reshape(max_pages, NH, page, D)
                per_layer.append(orc.f16_values(np.stack(
                    [pool[p // page, :, p % page, :] for p in range(length)], axis=1)))
            out.append(per_layer)
        return out

    P = len(prompt)
    t = np.tile(tables, (1, P, 1)).reshape(L, P, max_pages)
    logits, nxt = orc.decoder_step(m, cfg, k, v, page, max_pages, t, np.asarray(prompt, np.int32),
                                   np.arange(1, P + 1))
    out = [(logits, nxt, *caches(P))]
    for s, token in enumerate(decode_tokens):
        lg, nx = orc.decoder_step(m, cfg, k, v, page, max_pages, tables, np.array([token]),
                                  np.array([P + s + 1]))
        out.append((lg, nx, *caches(P + s + 1)))
    return out


def mha_kv_reference(x_q, x_k, x_v, wq, wk, wv, wo, heads, past=None):
    """float64 MultiHeadAttentionKVCache.forward (workloads/pytorch/KVCache.py):
    q/k/v projections, split heads, append to the past caches, softmax over
    every cached position (no mask), o projection.  x_* [seq, dim]; caches
    [heads, length, D]."""
    seq, dim = x_q.shape
    d = dim // heads
    split = lambda x: x.reshape(seq, heads, d).transpose(1, 0, 2)  # noqa: E731
    q, k, v = split(x_q @ wq.T), split(x_k @ wk.T), split(x_v @ wv.T)
    if past is not None:
        k = np.concatenate([past[0], k], axis=1)
        v = np.concatenate([past[1], v], axis=1)
    s = q @ k.transpose(0, 2, 1) / np.sqrt(d)
    s = np.exp(s - s.max(axis=-1, keepdims=True))
    s /= s.sum(axis=-1, keepdims=True)
    out = (s @ v).transpose(1, 0, 2).reshape(seq, dim) @ wo.T
    return out, (k, v)


def kv_workload(seed: int, heads=4, head_dim=16, prefill=7, decode=8):
    """The KV export's shapes (export_kv_cache.py:_make_references) with
    seeded inputs and weights ~ U(-1/sqrt(dim), 1/sqrt(dim)) as nn.Linear."""
    rng = np.random.default_rng(seed)
    dim = heads * head_dim
    bound = 1.0 / np.sqrt(dim)
    wq, wk, wv, wo = (rng.uniform(-bound, bound, (dim, dim)) for _ in range(4))
    xq, xk, xv = (rng.standard_normal((prefill, dim)) for _ in range(3))
    out, cache = mha_kv_reference(xq, xk, xv, wq, wk, wv, wo, heads)
    config = dict(batch=1, heads=heads, head_dimension=head_dim, capacity=prefill + decode,
                  prefill_length=prefill, decode_count=decode)
    tensors = {"query_weight": wq, "key_weight": wk, "value_weight": wv, "output_weight": wo,
               "prefill_query": xq, "prefill_key": xk, "prefill_value": xv,
               "prefill_output": out, "prefill_key_cache": cache[0],
               "prefill_value_cache": cache[1]}
    steps = []
    for _ in range(decode):
        sq, sk, sv = (rng.standard_normal((1, dim)) for _ in range(3))
        out, cache = mha_kv_reference(sq, sk, sv, wq, wk, wv, wo, heads, cache)
        steps.append(dict(query=sq, key=sk, value=sv, output=out, key_cache=cache[0],
                          value_cache=cache[1]))
    return config, tensors, steps
