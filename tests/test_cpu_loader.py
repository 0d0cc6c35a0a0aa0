"""What Engine::load_from refuses before it opens a device, without a GPU: the counterpart of
x0ne-core/oracle/tests/cpu_config.rs and cpu_safetensors.rs. A config the kernels do not serve,
a context out of range, a checkpoint that is not the config's, or a file whose header lies is a
FormatError; a load that passes every check ends on the missing device (GpuError) here, and loads
on a machine with a GPU. Nothing is ever another error or a crash."""
import json
import random

import numpy as np
import pytest

from common import reference_tensors, safetensors_bytes, tiny


def dense() -> dict:
    """cpu_config.rs:15-35"""
    return {"model_type": "qwen3", "dtype": "bfloat16", "hidden_act": "silu", "attention_bias": False,
            "hidden_size": 64, "intermediate_size": 96, "num_hidden_layers": 2, "num_attention_heads": 4,
            "num_key_value_heads": 2, "head_dim": 128, "vocab_size": 384, "max_position_embeddings": 2048,
            "rms_norm_eps": 1e-6, "rope_theta": 1000000.0, "tie_word_embeddings": False,
            "architectures": ["Qwen3ForCausalLM"], "use_cache": True}


SIZES = ["hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
         "head_dim", "vocab_size", "max_position_embeddings"]


@pytest.fixture(scope="module")
def checkpoint():
    cfg = tiny(2, 4, 2, False)
    return safetensors_bytes(reference_tensors(cfg, 41))


def load(config, file, max_ctx=64, files=None):
    from x0ne_core import Engine, EngineOptions
    text = config if isinstance(config, str) else json.dumps(config)
    return Engine.load_from(text, files if files is not None else {"model.safetensors": file},
                            EngineOptions(max_ctx=max_ctx))


def passed_the_checks(what, config, file, max_ctx=64, files=None):
    from x0ne_core import GpuError
    try:
        e = load(config, file, max_ctx, files)
    except GpuError:
        return
    e.close()  # a GPU is here: it loaded


def refused(what, config, file, max_ctx=64, files=None):
    from x0ne_core import FormatError
    with pytest.raises(FormatError):
        load(config, file, max_ctx, files)


def with_(key, value, base=None):
    v = dict(base or dense())
    v[key] = value
    return v


def without(key):
    v = dense()
    del v[key]
    return v


def test_the_model_itself_passes_the_checks(checkpoint):
    passed_the_checks("the model", dense(), checkpoint)
    passed_the_checks("the whole context", dense(), checkpoint, 2048)
    passed_the_checks("a context of one", dense(), checkpoint, 1)


def test_a_size_that_is_not_a_positive_integer_is_refused(checkpoint):
    bad = ["0", "-1", "-0", "1.0", "1.5", "1e3", '"64"', "null", "true", "[64]", "{}", "18446744073709551616",
           "1e400", "-9223372036854775808"]
    base = json.dumps(dense(), separators=(",", ":"))
    for key in SIZES:
        refused(f"{key} missing", without(key), checkpoint)
        for value in bad:
            text = base.replace(f'"{key}":{json.dumps(dense()[key])}', f'"{key}":{value}', 1)
            assert f'"{key}":{value}' in text
            refused(f"{key} = {value}", text, checkpoint)
    for key in ["rms_norm_eps", "rope_theta"]:
        refused(f"{key} missing", without(key), checkpoint)
        for value in [0, 0.0, -1e-6, "1e-6", None, False, [1.0]]:
            refused(f"{key} = {value}", with_(key, value), checkpoint)
        for value in ["NaN", "Infinity", "-Infinity", "1e999", "nan", "inf"]:
            text = base.replace(f'"{key}":{json.dumps(dense()[key])}', f'"{key}":{value}', 1)
            assert value in text
            refused(f"{key} = {value}", text, checkpoint)


def test_a_model_this_engine_does_not_implement_is_refused(checkpoint):
    for key, values in [("model_type", ["qwen2", "qwen3_moe", "Qwen3", "", None, 3]),
                        ("dtype", ["float32", "float16", "bf16", "", None, 16]),
                        ("hidden_act", ["gelu", "relu", "SiLU", None, ["silu"]]),
                        ("attention_bias", [True, 1, "false", 0]),
                        ("use_sliding_window", [True, 4096]),
                        ("rope_scaling", [{"type": "yarn", "factor": 4.0}, True, {}]),
                        ("tie_word_embeddings", ["true", 1, 0, None, []])]:
        for value in values:
            refused(f"{key} = {value}", with_(key, value), checkpoint)
    refused("model_type missing", without("model_type"), checkpoint)
    refused("hidden_act missing", without("hidden_act"), checkpoint)
    refused("no dtype at all", without("dtype"), checkpoint)
    v = dense()
    v["torch_dtype"] = "bfloat16"
    v["dtype"] = "float32"
    refused("dtype float32 over torch_dtype bfloat16", v, checkpoint)
    for q, kv in [(4, 3), (2, 4), (5, 2), (1, 2), (7, 3)]:
        refused(f"{q} heads over {kv}", with_("num_key_value_heads", kv, with_("num_attention_heads", q)), checkpoint)
    for odd in [1, 3, 127, 129, 64, 256]:
        refused(f"head_dim {odd}", with_("head_dim", odd), checkpoint)
    refused("a vocabulary past u32", with_("vocab_size", 1 << 32), checkpoint)
    for text in ["", " ", "null", "[]", '"qwen3"', "42", "{", "{}", '{"model_type":"qwen3"}', "﻿{}"]:
        refused(repr(text), text, checkpoint)


def test_a_config_that_differs_from_its_checkpoint_is_refused(checkpoint):
    """cpu_config.rs:500-568"""
    refused("max_ctx 0", dense(), checkpoint, 0)
    refused("max_ctx past the positions", dense(), checkpoint, 2049)
    refused("max_ctx u64 max", dense(), checkpoint, 2 ** 64 - 1)
    for key, value in [("head_dim", 64), ("head_dim", 256), ("hidden_size", 60), ("hidden_size", 68),
                       ("hidden_size", 72), ("intermediate_size", 104), ("num_hidden_layers", 1),
                       ("num_hidden_layers", 3), ("num_attention_heads", 2), ("num_attention_heads", 8),
                       ("vocab_size", 383), ("vocab_size", 385), ("tie_word_embeddings", True),
                       ("model_type", "qwen2"), ("dtype", "float32")]:
        refused(f"{key} = {value}", with_(key, value), checkpoint)
    refused("a truncated checkpoint", dense(), checkpoint[:-2])
    other = safetensors_bytes(reference_tensors(tiny(1, 4, 2, False), 43))
    refused("the checkpoint of a one-layer model", dense(), other)
    refused("no checkpoint", dense(), b"")
    refused("no file at all", dense(), None, files={})


def load_opts(config, file, **opts):
    from x0ne_core import Engine, EngineOptions
    return Engine.load_from(json.dumps(config), {"model.safetensors": file}, EngineOptions(**opts))


def test_a_kv_plane_past_the_attention_kernels_addressing_is_refused_before_the_device(checkpoint):
    """The attention kernels address one layer's K (or V) plane, every sequence's pages, by 32-bit
    byte offsets below 0xFFFFFFF0. This model keeps 2 kv heads x 128 dims x 2 bytes = 512 bytes
    per position and plane, so 64 sequences of 131072 positions need a 2^32-byte plane: refused
    (FormatError, before any device work) rather than loaded with offsets that would wrap onto
    another sequence's pages. 63 sequences (4,227,858,432 bytes) pass the checks; so do 64 of
    131056 (4,294,443,008 bytes, the largest whole-page context below the limit)."""
    from x0ne_core import FormatError, GpuError, NotImplementedFeature
    big = with_("max_position_embeddings", 1 << 17)
    with pytest.raises(FormatError, match="KV plane"):
        load_opts(big, checkpoint, max_ctx=1 << 17, max_batch=64)
    with pytest.raises(FormatError, match="KV plane"):
        load_opts(big, checkpoint, max_ctx=(1 << 17) - 15, max_batch=64)  # the same 8192 pages
    for ctx, batch in [((1 << 17), 63), ((1 << 17) - 16, 64)]:
        try:
            load_opts(big, checkpoint, max_ctx=ctx, max_batch=batch).close()
        except GpuError:
            pass
    with pytest.raises(FormatError):
        load_opts(dense(), checkpoint, max_ctx=64, max_batch=65)
    with pytest.raises(NotImplementedFeature):
        load_opts(dense(), checkpoint, max_ctx=64, max_batch=2, f64_sums=True)


def test_a_cut_or_corrupted_config_is_read_or_refused_never_a_crash(checkpoint):
    """cpu_config.rs:303-360: cut anywhere, or with bytes changed, a config is refused
    (FormatError) or read; one that is read and still the checkpoint's ends on the device."""
    from x0ne_core import FormatError, GpuError
    text = json.dumps(dense(), separators=(",", ":"))
    for n in range(len(text)):
        refused(f"cut at {n}", text[:n], checkpoint)
    rng = random.Random(31)
    outcomes = {"refused": 0, "passed": 0}
    for _ in range(3000):
        b = bytearray(text.encode())
        for _ in range(rng.randint(1, 3)):
            at = rng.randrange(len(b))
            r = rng.randrange(4)
            b[at] = (rng.choice(b"0123456789") if r == 0 else rng.choice(b'{}[],:"-+.eE ') if r == 1
                     else b[at] ^ (1 << rng.randrange(7)) if r == 2 else rng.randint(0x20, 0x7E))
        try:
            s = b.decode()
        except UnicodeDecodeError:
            continue
        try:
            e = load(s, checkpoint)
            e.close()
            outcomes["passed"] += 1
        except FormatError:
            outcomes["refused"] += 1
        except GpuError:
            outcomes["passed"] += 1
    print(f"MEASURE corrupted configs: {outcomes}")
    assert outcomes["refused"] > 100 and outcomes["passed"] > 20


# -------------------------------------------------------------------------------------------------
# safetensors (cpu_safetensors.rs)
# -------------------------------------------------------------------------------------------------


def header_and_data(file: bytes):
    n = int.from_bytes(file[:8], "little")
    return json.loads(file[8:8 + n]), file[8 + n:]


def rebuild(header: dict, data: bytes, pad_to=None) -> bytes:
    h = json.dumps(header).encode()
    return len(h).to_bytes(8, "little") + h + data


def test_a_checkpoint_truncated_at_any_length_is_refused(checkpoint):
    lengths = sorted(set(list(range(0, 64)) + list(range(64, len(checkpoint), 97)) + [len(checkpoint) - 1]))
    for n in lengths:
        refused(f"cut at {n}", dense(), checkpoint[:n])


def test_headers_that_lie_about_offsets_shapes_and_types_are_refused(checkpoint):
    header, data = header_and_data(checkpoint)
    name = "model.layers.0.self_attn.q_proj.weight"
    good = header[name]

    def lie(**kw):
        h = json.loads(json.dumps(header))
        h[name] = dict(good, **kw)
        return rebuild(h, data)

    a, b = good["data_offsets"]
    for offsets in [[a, b - 2], [a, b + 2], [a + 2, b], [b, a], [a, len(data) + 2], [-2, b], [a, 2 ** 64]]:
        refused(f"offsets {offsets}", dense(), lie(data_offsets=offsets))
    for shape in [[good["shape"][0], good["shape"][1] + 1], [good["shape"][1], good["shape"][0] + 1],
                  [good["shape"][0] * good["shape"][1]], [-1, 64], [2 ** 62, 4]]:
        refused(f"shape {shape}", dense(), lie(shape=shape))
    for dtype in ["F32", "F16", "BF8", "bf16", "", None, 16]:
        refused(f"dtype {dtype}", dense(), lie(dtype=dtype))
    # Two tensors over the same bytes, and a gap: neither is a well-formed file.
    h = json.loads(json.dumps(header))
    other = "model.layers.0.self_attn.k_proj.weight"
    h[other] = dict(h[other], data_offsets=h[name]["data_offsets"])
    refused("overlapping tensors", dense(), rebuild(h, data))
    # A header length past the file, or not valid JSON.
    n = int.from_bytes(checkpoint[:8], "little")
    for length in [n + 1, n - 1, len(checkpoint), 2 ** 63, 0]:
        refused(f"header length {length}", dense(), length.to_bytes(8, "little") + checkpoint[8:])
    refused("a header that is not JSON", dense(), (5).to_bytes(8, "little") + b"{oops" + data)


def test_random_corruption_of_a_checkpoint_never_crashes(checkpoint):
    from x0ne_core import FormatError, GpuError
    rng = random.Random(7)
    n = int.from_bytes(checkpoint[:8], "little")
    seen = {"refused": 0, "passed": 0}
    for _ in range(400):
        b = bytearray(checkpoint)
        for _ in range(rng.randint(1, 4)):
            at = rng.randrange(8 + n)  # the length and the header: the data bytes are any bytes
            b[at] = rng.randrange(256)
        try:
            load(dense(), bytes(b)).close()
            seen["passed"] += 1
        except FormatError:
            seen["refused"] += 1
        except GpuError:
            seen["passed"] += 1
    print(f"MEASURE corrupted checkpoints: {seen}")
    assert seen["refused"] > 100


def test_an_index_and_its_shards_must_agree():
    """cpu_safetensors.rs:509-615: a sharded checkpoint over an index."""
    cfg = tiny(2, 4, 2, False)
    t = reference_tensors(cfg, 41)
    names = list(t)
    first = {k: t[k] for k in names[: len(names) // 2]}
    second = {k: t[k] for k in names[len(names) // 2:]}
    files = {"a.safetensors": safetensors_bytes(first), "b.safetensors": safetensors_bytes(second)}
    index = {"metadata": {}, "weight_map": {**{k: "a.safetensors" for k in first},
                                            **{k: "b.safetensors" for k in second}}}
    from x0ne_core import Engine, EngineOptions, FormatError, GpuError

    def go(idx, fs):
        return Engine.load_from(json.dumps(dense()), fs, EngineOptions(max_ctx=64), json.dumps(idx))

    try:
        go(index, files).close()
    except GpuError:
        pass
    passed = {"the files swapped": {"b.safetensors": files["b.safetensors"], "a.safetensors": files["a.safetensors"]}}
    for what, fs in passed.items():
        try:
            go(index, fs).close()
        except GpuError:
            pass
    wrong = json.loads(json.dumps(index))
    wrong["weight_map"][names[0]] = "b.safetensors"
    missing = json.loads(json.dumps(index))
    del missing["weight_map"][names[-1]]
    extra = json.loads(json.dumps(index))
    extra["weight_map"]["model.extra.weight"] = "b.safetensors"
    a, b = files["a.safetensors"], files["b.safetensors"]
    cases = [("a tensor listed in the other shard", wrong, files),
             ("a tensor the index does not list", missing, files),
             ("a tensor the shards do not hold", extra, files),
             ("a shard missing", index, {"a.safetensors": a}),
             ("a file the index does not name", index, {"a.safetensors": a, "c.safetensors": b}),
             ("an extra file", index, {"a.safetensors": a, "b.safetensors": b, "c.safetensors": b}),
             ("no file", index, {}),
             ("the shards exchanged", index, {"a.safetensors": b, "b.safetensors": a}),
             ("a tensor held by two shards", index, {"a.safetensors": a, "b.safetensors": a}),
             ("a truncated shard", index, {"a.safetensors": a[:-1], "b.safetensors": b})]
    for what, idx, fs in cases:
        with pytest.raises(FormatError):
            go(idx, fs)
    for bad in ["{}", "[]", "", '{"weight_map":[]}', '{"weight_map":null}', '{"weight_map":{"a.weight":1}}',
                '{"weight_map":{"a.weight":null}}', '{"weight_map":{"a.weight":["a.safetensors"]}}',
                '{"weight_map":{"a.weight":"a.safetensors"}']:
        with pytest.raises(FormatError):
            Engine.load_from(json.dumps(dense()), files, EngineOptions(max_ctx=64), bad)
    # Without an index: exactly one file.
    with pytest.raises(FormatError):
        Engine.load_from(json.dumps(dense()), files, EngineOptions(max_ctx=64))


def load_dir(path, max_ctx=64):
    from x0ne_core import Engine, EngineOptions
    return Engine.load(str(path), EngineOptions(max_ctx=max_ctx))


def dir_passed_the_checks(path, max_ctx=64):
    from x0ne_core import GpuError
    try:
        e = load_dir(path, max_ctx)
    except GpuError:
        return
    e.close()


def test_a_model_directory_is_refused_on_what_it_lacks(checkpoint, tmp_path):
    """cpu_config.rs:569-612: Engine::load on a directory, the refusals of the in-memory load read
    from disk; no config.json is an I/O error."""
    from x0ne_core import FormatError, IoError
    with pytest.raises(IoError):
        load_dir(tmp_path)
    with pytest.raises(IoError):
        load_dir(tmp_path / "absent")
    (tmp_path / "config.json").write_text("{")
    with pytest.raises(FormatError):
        load_dir(tmp_path)
    (tmp_path / "config.json").write_text(json.dumps(dense()))
    with pytest.raises(FormatError):  # no weights
        load_dir(tmp_path)
    (tmp_path / "model.safetensors").write_bytes(checkpoint[: len(checkpoint) // 2])
    with pytest.raises(FormatError):
        load_dir(tmp_path)
    (tmp_path / "model.safetensors").write_bytes(checkpoint)
    with pytest.raises(FormatError):
        load_dir(tmp_path, max_ctx=0)
    dir_passed_the_checks(tmp_path)


def test_a_model_directory_is_one_file_or_an_index(checkpoint, tmp_path):
    """cpu_safetensors.rs:691-758 (Safetensors::open_dir): one file or an index, never both, never
    neither; every truncation on disk refused, the empty file included; an index's shard read
    like the single file. The 64 GiB per-file cap itself is not exercised here."""
    from x0ne_core import Error, FormatError
    (tmp_path / "config.json").write_text(json.dumps(dense()))
    single = tmp_path / "model.safetensors"
    single.write_bytes(checkpoint)
    dir_passed_the_checks(tmp_path)
    (tmp_path / "model.safetensors.index.json").write_text('{"weight_map":{}}')
    with pytest.raises(FormatError):  # both present
        load_dir(tmp_path)
    (tmp_path / "model.safetensors.index.json").unlink()
    for cut in [0, 1, 7, 8, 9, len(checkpoint) // 2, len(checkpoint) - 1]:
        single.write_bytes(checkpoint[:cut])
        with pytest.raises(FormatError):
            load_dir(tmp_path)
    single.unlink()
    (tmp_path / "s.safetensors").write_bytes(checkpoint)
    header_len = int.from_bytes(checkpoint[:8], "little")
    names = [k for k in json.loads(checkpoint[8:8 + header_len]) if k != "__metadata__"]
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {n: "s.safetensors" for n in names}}))
    dir_passed_the_checks(tmp_path)
    (tmp_path / "s.safetensors").write_bytes(b"")
    with pytest.raises(Error):
        load_dir(tmp_path)


def test_a_shard_name_is_a_plain_file_name(checkpoint, tmp_path):
    """cpu_safetensors.rs:616-689 (st.rs:83-87): an index naming a path, a parent, a hidden file or
    a directory part is a format error, on disk and in memory; plain names that are not a
    readable shard are an error of the file system or of the format, never a crash."""
    from x0ne_core import Engine, EngineOptions, Error, FormatError
    model = tmp_path / "model"
    outside = tmp_path / "outside"
    model.mkdir()
    outside.mkdir()
    (model / "config.json").write_text(json.dumps(dense()))
    (model / "inside.safetensors").write_bytes(checkpoint)
    (outside / "secret.safetensors").write_bytes(checkpoint)
    (model / "sub").mkdir()
    (model / "sub" / "deep.safetensors").write_bytes(checkpoint)
    header_len = int.from_bytes(checkpoint[:8], "little")
    names = [k for k in json.loads(checkpoint[8:8 + header_len]) if k != "__metadata__"]

    def write_index(shard):
        text = json.dumps({"weight_map": {n: shard for n in names}})
        (model / "model.safetensors.index.json").write_text(text)
        return text

    write_index("inside.safetensors")
    dir_passed_the_checks(model)
    for name in [str(outside / "secret.safetensors"), "../outside/secret.safetensors", "sub/deep.safetensors",
                 "sub\\deep.safetensors", "./inside.safetensors", ".hidden.safetensors", "..", ".", "/etc/hostname"]:
        text = write_index(name)
        with pytest.raises(FormatError):
            load_dir(model)
        with pytest.raises(FormatError):
            Engine.load_from(json.dumps(dense()), {name: checkpoint}, EngineOptions(max_ctx=64), text)
    for name in ["", "absent.safetensors", "sub", "inside.safetensors\0x"]:
        write_index(name)
        with pytest.raises(Error):
            load_dir(model)


def moe_config(base=None) -> dict:
    """cpu_config.rs:37-46"""
    v = dict(base or dense())
    v.update({"model_type": "qwen3_moe", "decoder_sparse_step": 1, "norm_topk_prob": True, "num_experts": 8,
              "num_experts_per_tok": 2, "moe_intermediate_size": 16, "mlp_only_layers": []})
    return v


def moe_checkpoint(cfg_json: dict, seed: int = 5) -> bytes:
    """A Qwen3-MoE checkpoint of cfg_json's shapes: the dense model's attention, norms and
    vocabulary, and per layer the router and every expert's gate, up and down projections."""
    c = cfg_json
    h, layers, experts, mi = c["hidden_size"], c["num_hidden_layers"], c["num_experts"], c["moe_intermediate_size"]
    base = reference_tensors(tiny(layers, c["num_attention_heads"], c["num_key_value_heads"], False), seed)
    out = {k: v for k, v in base.items() if ".mlp." not in k}
    g = np.random.default_rng(seed)

    def bits(*shape):
        return shape, (g.integers(0, 1 << 14, size=int(np.prod(shape))) | 0x3C00).astype(np.uint16)

    for l in range(layers):
        out[f"model.layers.{l}.mlp.gate.weight"] = bits(experts, h)
        for e in range(experts):
            out[f"model.layers.{l}.mlp.experts.{e}.gate_proj.weight"] = bits(mi, h)
            out[f"model.layers.{l}.mlp.experts.{e}.up_proj.weight"] = bits(mi, h)
            out[f"model.layers.{l}.mlp.experts.{e}.down_proj.weight"] = bits(h, mi)
    return safetensors_bytes(out)


@pytest.fixture(scope="module")
def moe_file():
    return moe_checkpoint(moe_config())


def test_a_qwen3_moe_config_reads_strictly(moe_file):
    """cpu_config.rs:362-453 through Engine::load_from: the config itself passes the checks; every
    value the reader refuses (shared experts, a sparse step other than 1, dense layers, top-k not
    renormalised, sizes that are not positive integers, more experts per token than experts) is a
    format error, and so is each required key missing; the optional keys may be null or absent."""
    passed_the_checks("the MoE config", moe_config(), moe_file)
    for key, values in [("shared_expert_intermediate_size", [64, 0, False]), ("n_shared_experts", [1, 0]),
                        ("decoder_sparse_step", [2, 0, None, "1"]), ("mlp_only_layers", [[0], 0, {}, False]),
                        ("norm_topk_prob", [False, None, 1, "true"]),
                        ("num_experts", [0, 1, -8, 8.5, 1 << 32, None]), ("num_experts_per_tok", [0, 9, -1, "2"]),
                        ("moe_intermediate_size", [0, -16, 16.5, None])]:
        for value in values:
            refused(f"{key} = {value}", with_(key, value, moe_config()), moe_file)
    for key in ["decoder_sparse_step", "norm_topk_prob", "num_experts", "num_experts_per_tok",
                "moe_intermediate_size"]:
        v = moe_config()
        del v[key]
        refused(f"{key} missing", v, moe_file)
    for key in ["mlp_only_layers", "shared_expert_intermediate_size", "n_shared_experts"]:
        passed_the_checks(f"{key} null", with_(key, None, moe_config()), moe_file)
        v = moe_config()
        v.pop(key, None)
        passed_the_checks(f"{key} absent", v, moe_file)


def test_read_any_tells_dense_from_moe_and_refuses_the_rest(checkpoint, moe_file):
    """cpu_config.rs:455-475 and :548-565: other model types are refused; a MoE config without its
    fields, a MoE config over dense weights, a dense config over MoE weights, and the kernels'
    limits (1025 experts, 33 per token, a width that is not a multiple of 8) are format errors."""
    for model_type in ["qwen2", "qwen2_moe", "llama", "", "qwen3_moe "]:
        refused(model_type, with_("model_type", model_type, moe_config()), moe_file)
    refused("a MoE without its fields", with_("model_type", "qwen3_moe"), checkpoint)
    refused("a MoE config over dense weights", moe_config(), checkpoint)
    refused("a dense config over MoE weights", dense(), moe_file)
    for key, value in [("num_experts", 1025), ("num_experts_per_tok", 33), ("moe_intermediate_size", 12)]:
        big = with_("num_experts", 1024, moe_config())
        refused(f"{key} = {value}", with_(key, value, big), moe_file)
    for bad in ["", "[]"]:
        refused(f"config {bad!r}", bad, moe_file)


def test_the_accumulation_option_is_checked_before_the_device(checkpoint):
    """x0ne_engine_options.sums: 0 (the default: the exact mode where the engine has its kernels,
    else f32), 1 (f64, refused with X0NE_ERR_NOT_IMPLEMENTED where there are none: batched
    engines), 2 (f32); any other value is a format error. All of it before any device work, so
    without a GPU an accepted load ends in GpuError."""
    import ctypes as C
    from x0ne_core import FormatError, GpuError, NotImplementedFeature
    from x0ne_core import _lib
    from x0ne_core.engine import SUMS_DEFAULT, SUMS_F32, SUMS_F64
    lib = _lib.lib()
    cfg = json.dumps(dense()).encode()
    names = (C.c_char_p * 1)(b"model.safetensors")
    buf = C.create_string_buffer(checkpoint, len(checkpoint))
    data = (C.c_void_p * 1)(C.addressof(buf))
    lens = (C.c_uint64 * 1)(len(checkpoint))

    def status(sums, max_batch=0):
        opts = _lib.EngineOptionsC(64, 0, sums, 0, max_batch, 0)
        out = C.c_void_p()
        st = lib.x0ne_engine_load_from(cfg, 1, names, data, lens, None, C.byref(opts), C.byref(out))
        if out.value:
            lib.x0ne_engine_free(out)
        return st
    assert status(3) == _lib.ERR_FORMAT
    assert status(0xFFFFFFFF) == _lib.ERR_FORMAT
    assert status(SUMS_F64, max_batch=2) == _lib.ERR_NOT_IMPLEMENTED
    for sums, batch in [(SUMS_DEFAULT, 0), (SUMS_DEFAULT, 2), (SUMS_F64, 1), (SUMS_F32, 2)]:
        assert status(sums, batch) in (_lib.OK, _lib.ERR_GPU), (sums, batch)
    with pytest.raises(FormatError):
        load_opts(dense(), checkpoint, max_ctx=64, max_batch=65, f64_sums=None)
    with pytest.raises(NotImplementedFeature):
        load_opts(dense(), checkpoint, max_ctx=64, max_batch=2, f64_sums=True)
    for f64 in (None, False):
        try:
            load_opts(dense(), checkpoint, max_ctx=64, max_batch=2, f64_sums=f64).close()
        except GpuError:
            pass
