"""CPU: the `.tmc` importers (DecoderLLMImporter.cpp:154-279,
KVCacheImporter.cpp:95-200) read back exactly what the manifest writer put
in, derive the plan as the reference does, and refuse malformed manifests
with the reference's messages."""
import os

import numpy as np
import pytest

from tests import tmc_manifest as tm


def _random_decoder_tensors(config, seed=3):
    rng = np.random.default_rng(seed)
    H, I, V, L = (config["hidden_size"], config["intermediate_size"], config["vocabulary_size"],
                  config["layers"])
    C, P, D = config["capacity"], config["prefill_length"], H // config["heads"]
    t = {"embedding.weight": rng.standard_normal(V * H), "final_norm.weight": rng.random(H),
         "lm_head.weight": rng.standard_normal(V * H), "rope.cosine": rng.random(C * D // 2),
         "rope.sine": rng.random(C * D // 2)}
    for l in range(L):
        for name, n in (("input_norm", H), ("q", H * H), ("k", H * H), ("v", H * H),
                        ("o", H * H), ("post_norm", H), ("gate", I * H), ("up", I * H),
                        ("down", H * I)):
            t[f"layer{l}.{name}.weight"] = rng.standard_normal(n)
    for prefix, seq, length in [("prefill", P, P)] + [(f"decode{s}", 1, P + s + 1)
                                                     for s in range(config["decode_count"])]:
        t[f"{prefix}.tokens"] = rng.integers(0, V, seq)
        t[f"{prefix}.logits"] = rng.standard_normal(seq * V)
        t[f"{prefix}.next_tokens"] = rng.integers(0, V, 1)
        for l in range(L):
            t[f"{prefix}.layer{l}.key_cache"] = rng.standard_normal(config["heads"] * length * D)
            t[f"{prefix}.layer{l}.value_cache"] = rng.standard_normal(config["heads"] * length * D)
    return {k: np.asarray(v, np.float32) for k, v in t.items()}


def _f32(x):
    return np.asarray(x, np.float32)


def test_decoder_manifest_round_trip(host, tmp_path):
    config = tm.decoder_config(decode=3)
    tensors = _random_decoder_tensors(config)
    path = tm.write_decoder_manifest(tmp_path / "d.tmc", config, tensors, dtype=("F16", "BF16"))
    w, err = host.import_decoder_llm_workload(str(path))
    assert err == "" and w is not None
    plan = w.plan
    assert (plan.attention.heads, plan.attention.head_dimension, plan.attention.capacity,
            plan.attention.prefill_length) == (4, 16, 32, 8)
    assert (plan.layer_count, plan.intermediate_size, plan.vocabulary_size) == (2, 128, 128)
    assert plan.attention.threads_per_threadgroup == 128
    assert abs(plan.rms_norm_epsilon - 1e-5) < 1e-12
    assert w.requested_storage_dtype == host.DType.Float16
    assert plan.attention.dtype == host.DType.BFloat16  # the effective dtype of version 2
    assert w.decode_count == 3 and w.model_name == "DecoderOnlyLLM"
    assert np.array_equal(w.embedding_weight, tensors["embedding.weight"])
    assert np.array_equal(w.rope_sine, tensors["rope.sine"])
    assert np.array_equal(w.layers[1].down_weight, tensors["layer1.down.weight"])
    assert np.array_equal(w.layers[0].post_attention_norm_weight,
                          tensors["layer0.post_norm.weight"])
    assert np.array_equal(_f32(w.prefill.logits), tensors["prefill.logits"])
    assert np.array_equal(_f32(w.prefill.token_ids), tensors["prefill.tokens"])
    assert len(w.decode_steps) == 3
    assert np.array_equal(_f32(w.decode_steps[2].value_caches[1]),
                          tensors["decode2.layer1.value_cache"])
    assert w.decode_steps[2].key_caches[0].size == 4 * 11 * 16  # length P + 3


def test_decoder_manifest_dtype_forms(host, tmp_path):
    config = tm.decoder_config(decode=1)
    tensors = _random_decoder_tensors(config)
    # version 1 without DTYPE: fp32
    p = tm.write_decoder_manifest(tmp_path / "a.tmc", config, tensors, dtype=None, version=1)
    w, err = host.import_decoder_llm_workload(str(p))
    assert err == ""
    assert w.requested_storage_dtype == host.DType.Float32 and w.plan.attention.dtype == host.DType.Float32
    # version 1 with one DTYPE token: requested = effective
    p = tm.write_decoder_manifest(tmp_path / "b.tmc", config, tensors, dtype=("F16", None), version=1)
    w, err = host.import_decoder_llm_workload(str(p))
    assert err == "" and w.plan.attention.dtype == host.DType.Float16
    # threads double until they cover the head dimension (D = 256)
    big = tm.decoder_config(hidden=512, heads=2, decode=1)
    p = tm.write_decoder_manifest(tmp_path / "c.tmc", big, _random_decoder_tensors(big))
    w, err = host.import_decoder_llm_workload(str(p))
    assert err == "" and w.plan.attention.threads_per_threadgroup == 256


@pytest.mark.parametrize("case,message", [
    ("magic", "Invalid or unsupported decoder-only manifest header."),
    ("version", "Invalid or unsupported decoder-only manifest header."),
    ("missing", "Missing decoder-only tensor 'layer1.up.weight'."),
    ("count", "Invalid decoder-only tensor range for 'final_norm.weight'."),
    ("range", "Invalid decoder-only tensor range for 'lm_head.weight'."),
    ("duplicate", "Duplicate decoder-only tensor 'rope.sine'."),
    ("trailing", "Unexpected data after decoder-only END marker."),
    ("heads", "Decoder hidden size must be divisible by head count."),
    ("decode", "Decoder decode steps exceed cache capacity."),
    ("dtype", "Unsupported decoder-only dtype 'F8'."),
    ("payload", "Unable to open decoder-only payload"),
    ("aligned", "payload is not float32-aligned."),
])
def test_decoder_manifest_errors(host, tmp_path, case, message):
    config = tm.decoder_config(decode=1)
    tensors = _random_decoder_tensors(config)
    kwargs = {}
    if case == "missing":
        del tensors["layer1.up.weight"]
    elif case == "count":
        tensors["final_norm.weight"] = tensors["final_norm.weight"][:-1]
    elif case == "trailing":
        kwargs["extra_lines"] = ["surplus"]
    elif case == "heads":
        config["heads"] = 3
    elif case == "decode":
        config["decode_count"] = config["capacity"]
    elif case == "dtype":
        kwargs["dtype"] = ("F8", "F16")
    path = tm.write_decoder_manifest(tmp_path / "m.tmc", config, tensors, **kwargs)
    text = path.read_text()
    if case == "magic":
        text = text.replace("TMC_DECODER_LLM", "TMC_DECODER", 1)
    elif case == "version":
        text = text.replace("TMC_DECODER_LLM 2", "TMC_DECODER_LLM 3", 1)
    elif case == "range":
        line = next(l for l in text.splitlines() if l.startswith('TENSOR "lm_head.weight"'))
        name, _, count = line.rsplit(" ", 2)
        text = text.replace(line, f"{name} 999999999 {count}")
    elif case == "duplicate":
        line = next(l for l in text.splitlines() if l.startswith('TENSOR "rope.sine"'))
        text = text.replace(line, line + "\n" + line).replace(
            f"TENSORS {len(tensors)}", f"TENSORS {len(tensors) + 1}")
    elif case == "payload":
        (tmp_path / "m.tmc.bin").unlink()
    elif case == "aligned":
        with open(tmp_path / "m.tmc.bin", "ab") as f:
            f.write(b"\0\0")
    path.write_text(text)
    w, err = host.import_decoder_llm_workload(str(path))
    assert w is None and message in err, err
    w, err = host.import_decoder_llm_workload(str(tmp_path / "absent.tmc"))
    assert w is None and "Unable to open decoder-only manifest" in err


def test_kv_manifest_round_trip_and_reference(host, tmp_path):
    config, tensors, steps = tm.kv_workload(5)
    path = tm.write_kv_manifest(tmp_path / "kv.tmc", config, tensors, steps)
    w, err = host.import_kv_cache_workload(str(path))
    assert err == "" and w is not None
    plan = w.plan
    assert (plan.batch, plan.heads, plan.head_dimension, plan.capacity, plan.prefill_length) == \
        (1, 4, 16, 15, 7)
    assert plan.dtype == host.DType.Float32
    assert np.array_equal(w.output_weight, _f32(tensors["output_weight"]).ravel())
    assert np.array_equal(_f32(w.prefill.value_cache), _f32(tensors["prefill_value_cache"]).ravel())
    assert len(w.decode_steps) == 8
    assert np.array_equal(_f32(w.decode_steps[7].key_cache), _f32(steps[7]["key_cache"]).ravel())
    # the numpy reference itself: a decode step equals the prefill of the
    # whole sequence's last row (attention over every cached position)
    x = [np.concatenate([tensors[f"prefill_{n}"], steps[0][n]]) for n in ("query", "key", "value")]
    full, _ = tm.mha_kv_reference(*x, tensors["query_weight"], tensors["key_weight"],
                                  tensors["value_weight"], tensors["output_weight"], 4)
    assert np.allclose(full[-1], steps[0]["output"][0], atol=1e-12)


@pytest.mark.parametrize("case,message", [
    ("magic", "Invalid or unsupported KV cache manifest header."),
    ("steps", "KV cache CONFIG and STEPS counts disagree."),
    ("order", "KV cache decode steps are out of order."),
    ("missing", "Missing KV cache tensor 'prefill_output'."),
    ("count", "Invalid KV cache tensor range for 'key_weight'."),
    ("capacity", "Decode steps exceed the configured cache capacity."),
])
def test_kv_manifest_errors(host, tmp_path, case, message):
    config, tensors, steps = tm.kv_workload(6, decode=3)
    kwargs = {}
    if case == "steps":
        kwargs["declared_steps"] = 2
    elif case == "order":
        kwargs["step_indices"] = [0, 2, 1]
    elif case == "missing":
        del tensors["prefill_output"]
    elif case == "count":
        tensors["key_weight"] = tensors["key_weight"][:-1]
    elif case == "capacity":
        config["capacity"] = config["prefill_length"] + 1
    path = tm.write_kv_manifest(tmp_path / "kv.tmc", config, tensors, steps, **kwargs)
    if case == "magic":
        path.write_text(path.read_text().replace("TMC_KV_CACHE 1", "TMC_KV_CACHE 2", 1))
    w, err = host.import_kv_cache_workload(str(path))
    assert w is None and message in err, err


GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("fixture,requested,effective", [
    ("decoder_llm_fp16_seed11.tmc", "Float16", "Float16"),
    ("decoder_llm_fp32_seed11.tmc", "Float32", "Float32"),
])
def test_reference_exporter_decoder_manifest(host, fixture, requested, effective):
    """Manifests written by the reference's own exporter
    (tools/export_decoder_llm.py, seed 11, default shape;
    tests/golden/make_tmc_golden.py) import with this build's importer:
    version 2 header, CONFIG, DTYPE requested/effective, every tensor range,
    the prefill and 8 decode references.  Properties the exporter's PyTorch
    run fixes: each reference's next token is the argmax of its last logits
    row, each decode step's input token is the previous step's next token,
    caches grow by one position per step, and fp16 exports store
    fp16-representable weights."""
    w, err = host.import_decoder_llm_workload(os.path.join(GOLDEN, fixture))
    assert err == "" and w is not None, err
    plan = w.plan
    assert w.model_name == "DecoderOnlyLLM"
    assert (plan.attention.batch, plan.attention.heads, plan.attention.head_dimension,
            plan.attention.capacity, plan.attention.prefill_length) == (1, 4, 16, 32, 8)
    assert (plan.layer_count, plan.intermediate_size, plan.vocabulary_size) == (2, 128, 128)
    assert abs(plan.rms_norm_epsilon - 1e-5) < 1e-12
    assert w.requested_storage_dtype == getattr(host.DType, requested)
    assert plan.attention.dtype == getattr(host.DType, effective)
    assert w.decode_count == 8 and len(w.decode_steps) == 8
    V, H = 128, 64
    assert w.embedding_weight.size == V * H and w.language_model_head_weight.size == V * H
    assert w.layers[1].down_weight.size == 128 * H
    if requested == "Float16":
        for arr in (w.embedding_weight, w.layers[0].query_weight, w.layers[1].down_weight):
            a = np.asarray(arr, np.float32)
            assert np.array_equal(a.astype(np.float16).astype(np.float32), a)
    logits = _f32(w.prefill.logits).reshape(8, V)
    assert int(w.prefill.next_token_ids[0]) == int(np.argmax(logits[-1]))
    previous = int(w.prefill.next_token_ids[0])
    for s, step in enumerate(w.decode_steps):
        assert int(step.token_ids[0]) == previous, s
        assert int(step.next_token_ids[0]) == int(np.argmax(_f32(step.logits))), s
        previous = int(step.next_token_ids[0])
        assert step.key_caches[0].size == 4 * (8 + s + 1) * 16
        # the prefix the step extends is the previous step's cache
        earlier = w.prefill if s == 0 else w.decode_steps[s - 1]
        n = 4 * (8 + s) * 16
        k_now = _f32(step.key_caches[1]).reshape(4, 8 + s + 1, 16)[:, :8 + s]
        k_before = _f32(earlier.key_caches[1]).reshape(4, 8 + s, 16)
        assert k_now.size == n and np.array_equal(k_now, k_before), s


def test_reference_exporter_kv_manifest(host):
    """The reference exporter's KV-cache manifest (tools/export_kv_cache.py)
    imports: CONFIG 1 4 16 15 7 8, ten tensors, eight steps whose caches
    extend the previous ones by one position."""
    w, err = host.import_kv_cache_workload(os.path.join(GOLDEN, "kv_cache.tmc"))
    assert err == "" and w is not None, err
    plan = w.plan
    assert (plan.batch, plan.heads, plan.head_dimension, plan.capacity, plan.prefill_length) == \
        (1, 4, 16, 15, 7)
    assert w.model_name == "MultiHeadAttentionKVCache"
    assert w.query_weight.size == 64 * 64 and w.prefill.output.size == 7 * 64
    assert len(w.decode_steps) == 8
    before = _f32(w.prefill.key_cache).reshape(4, 7, 16)
    for s, step in enumerate(w.decode_steps):
        now = _f32(step.key_cache).reshape(4, 8 + s, 16)
        assert np.array_equal(now[:, :7 + s], before), s
        before = now
