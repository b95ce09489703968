"""The C++ host layer (infer_amd/host/iq_host.h) through its test program
tests/cpp/test_host (built by __graft_entry__.build()):

* .llmq reading: QuantModel::load of a model directory written by the
  reference's own QuantWriter (tests/golden/tiny_model, see
  gen_tiny_model.py) yields every tensor with the reference's names, order,
  shapes and payload bytes (FNV-1a-64 against the fixture's manifest);
* .llmq writing: re-writing those tensors with our QuantWriter reproduces the
  reference's file byte for byte (src/quant.cpp:106-134 format);
* malformed containers throw;
* on the GPU: on-device quantize bit-exact, the QuantView launchers on every
  matrix of the tiny model (int8 / int4, T = 1, 3, 40) within the reference's
  5e-6 conditioning tolerance, the embedding gather exact.
"""
import json
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "cpp", "test_host")
TINY = os.path.join(HERE, "golden", "tiny_model")


def run(*args, timeout=120):
    if not os.path.exists(EXE):
        pytest.fail("tests/cpp/test_host is not built (run __graft_entry__.build())")
    r = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=timeout)
    return r.returncode, r.stdout, r.stderr


@pytest.mark.parametrize("kind,fname", [("int8", "model.q8.llmq"), ("int4", "model.q4.llmq")])
def test_llmq_read_matches_reference_writer(kind, fname):
    rc, out, err = run("dump", TINY, kind)
    assert rc == 0, out + err
    lines = out.strip().splitlines()
    assert lines[0] == "layers 2 tied 0 bias 1"
    manifest = json.load(open(os.path.join(TINY, "manifest.json")))[fname]
    assert len(lines) - 1 == len(manifest)
    for line, ref in zip(lines[1:], manifest):
        f = line.split()
        assert f[0] == ref["name"] and f[1] == ref["dtype"], (line, ref)
        if ref["dtype"] == "bf16":
            assert [int(f[2])] == ref["shape"] and f[4] == ref["data"], (line, ref)
        else:
            assert [int(f[2]), int(f[3])] == ref["shape"], (line, ref)
            assert f[4] == ref["q"] and f[5] == ref["scales"], (line, ref)
            if ref["dtype"] == "int4":
                assert f[6] == ref["zeros"], (line, ref)


@pytest.mark.parametrize("src", ["tiny_model/model.q8.llmq", "tiny_model/model.q4.llmq", "ref_small_int4.llmq"])
def test_llmq_write_is_byte_identical(src, tmp_path):
    path = os.path.join(HERE, "golden", src)
    out = str(tmp_path / "rt.llmq")
    rc, o, e = run("roundtrip", path, out)
    assert rc == 0, o + e
    assert open(out, "rb").read() == open(path, "rb").read()


def test_llmq_malformed_containers_throw(tmp_path):
    rc, out, err = run("errors", str(tmp_path))
    assert rc == 0, out + err


@pytest.mark.gpu
def test_host_launchers_on_gpu():
    print("test_host gpu", TINY, flush=True)
    rc, out, err = run("gpu", TINY, timeout=110)
    assert rc == 0, out + err


def _tiny_entries():
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from gen_tiny_model import fnv1a64, tiny_entries
    return tiny_entries(), fnv1a64


def test_tiny_model_sources_reproduce_the_fixture():
    """The seeded bf16 tensors of tests/golden/gen_tiny_model.py, packed by
    the oracle's quantiser (src/quant.cpp restated, pinned to the
    reference's vectors), hash to the manifest the reference's own writer
    recorded: they are the inputs the fixture files were made from."""
    import numpy as np
    from oracle import oracle as O
    entries, fnv = _tiny_entries()
    manifest = json.load(open(os.path.join(TINY, "manifest.json")))
    for kind, fname in ((0, "model.q8.llmq"), (1, "model.q4.llmq")):
        assert [e[1] for e in entries] == [m["name"] for m in manifest[fname]]
        for (typ, name, arr), ref in zip(entries, manifest[fname]):
            if typ == "v":
                assert fnv(arr.tobytes()) == ref["data"], name
            else:
                q, s, z = O.quantize(arr, kind)
                assert fnv(q.tobytes()) == ref["q"] and fnv(s.tobytes()) == ref["scales"], name
                if kind == 1:
                    assert fnv(z.tobytes()) == ref["zeros"], name


def _write_tensors(path, entries):
    import struct
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(entries)))
        for _, name, arr in entries:
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<I", arr.ndim))
            f.write(struct.pack(f"<{arr.ndim}q", *arr.shape))
            f.write(arr.astype("<u2").tobytes())


@pytest.mark.gpu
@pytest.mark.parametrize("kind,fname", [("int8", "model.q8.llmq"), ("int4", "model.q4.llmq")])
def test_quantize_model_on_gpu_writes_the_reference_file(kind, fname, tmp_path):
    """llm::quantize_model (tools/quantize.cpp:30-83's loop, packing on the
    GPU) over the tiny model's bf16 tensors writes the reference's own
    .llmq file byte for byte, and reports a worst group error within the
    quantiser's bounds: half a step for int8 (step = absmax / 127, its bf16
    rounding included: < 1/200 of absmax); for int4 a step of (hi - lo) / 15
    <= 2 absmax / 15 (half a step of rounding plus the zero point's)."""
    entries, _ = _tiny_entries()
    src = str(tmp_path / "tensors.bin")
    _write_tensors(src, entries)
    out = str(tmp_path / fname)
    print("qmodel", kind, flush=True)
    rc, o, e = run("qmodel", src, TINY, kind, out, timeout=110)
    assert rc == 0, o + e
    assert open(out, "rb").read() == open(os.path.join(TINY, fname), "rb").read()
    worst = float(o.split("worst group error")[1].split()[0])
    assert 0 < worst <= (1 / 200 if kind == "int8" else 2 / 15), worst


@pytest.mark.gpu
@pytest.mark.parametrize("kind,rows", [("int8", 1), ("int4", 1), ("int4", 3), ("int8", 12)])
def test_decode_step_through_the_host_layer(kind, rows, tmp_path):
    """The C++ host path end to end: quantize_model (GPU) writes a .llmq,
    QuantModel::load reads it, DevQuantModel uploads it, gpu::DecodeStep
    runs the chained decode step of one token per sequence for `rows`
    sequences (row b: token + 7 b); every row's logits match the oracle's
    float64 forward of src/forward.cpp on the dequantised weights
    (max |err| / max |ref| <= 1e-3)."""
    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(4242)
    H, I, nh, nkv, hd, V, L = 256, 512, 2, 1, 128, 300, 2
    cfg = {"architectures": ["Qwen2ForCausalLM"], "hidden_size": H, "intermediate_size": I,
           "num_attention_heads": nh, "num_key_value_heads": nkv, "num_hidden_layers": L, "vocab_size": V,
           "rope_theta": 1000000.0, "rms_norm_eps": 1e-6, "tie_word_embeddings": False}
    json.dump(cfg, open(tmp_path / "config.json", "w"))
    mat = lambda r, c, sd=0.05: O.seeded_bf16(rng, (r, c), sd)
    vec = lambda n, base=0.0: O.f32_to_bf16(base + rng.standard_normal(n).astype(np.float32) * np.float32(0.1))
    ents = [("m", "model.embed_tokens.weight", mat(V, H, 0.5)), ("m", "lm_head.weight", mat(V, H)),
            ("v", "model.norm.weight", vec(H, 1.0))]
    for i in range(L):
        p = f"model.layers.{i}."
        ents += [("m", p + "self_attn.q_proj.weight", mat(nh * hd, H)), ("m", p + "self_attn.k_proj.weight", mat(nkv * hd, H)),
                 ("m", p + "self_attn.v_proj.weight", mat(nkv * hd, H)), ("m", p + "self_attn.o_proj.weight", mat(H, nh * hd)),
                 ("m", p + "mlp.gate_proj.weight", mat(I, H)), ("m", p + "mlp.up_proj.weight", mat(I, H)),
                 ("m", p + "mlp.down_proj.weight", mat(H, I)), ("v", p + "input_layernorm.weight", vec(H, 1.0)),
                 ("v", p + "post_attention_layernorm.weight", vec(H, 1.0)), ("v", p + "self_attn.q_proj.bias", vec(nh * hd)),
                 ("v", p + "self_attn.k_proj.bias", vec(nkv * hd)), ("v", p + "self_attn.v_proj.bias", vec(nkv * hd))]
    _write_tensors(str(tmp_path / "tensors.bin"), ents)
    token = 123
    out = str(tmp_path / "logits.bin")
    print("host chain", kind, rows, flush=True)
    os.environ["IQ_TEST_ROWS"] = str(rows)
    try:
        rc, o, e = run("chain", str(tmp_path / "tensors.bin"), str(tmp_path), kind, str(token), out, timeout=110)
    finally:
        del os.environ["IQ_TEST_ROWS"]
    assert rc == 0, o + e
    got = np.fromfile(out, dtype=np.float32).astype(np.float64)
    k = 1 if kind == "int4" else 0
    t = {name: arr for _, name, arr in ents}

    def dq(name):
        a = t[name]
        q, s, z = O.quantize(a, k)
        return O.dequant_matrix(q, s, z, k, a.shape[0], a.shape[1])

    model = {"cfg": dict(hidden=H, heads=nh, kv_heads=nkv, head_dim=hd, eps=1e-6),
             "embed_dq": dq("model.embed_tokens.weight"), "head_dq": dq("lm_head.weight"),
             "final_norm": t["model.norm.weight"], "layers": []}
    for i in range(L):
        p = f"model.layers.{i}."
        model["layers"].append({
            "q": dq(p + "self_attn.q_proj.weight"), "k": dq(p + "self_attn.k_proj.weight"),
            "v": dq(p + "self_attn.v_proj.weight"), "o": dq(p + "self_attn.o_proj.weight"),
            "gate": dq(p + "mlp.gate_proj.weight"), "up": dq(p + "mlp.up_proj.weight"),
            "down": dq(p + "mlp.down_proj.weight"), "input_ln": t[p + "input_layernorm.weight"],
            "post_ln": t[p + "post_attention_layernorm.weight"], "q_b": t[p + "self_attn.q_proj.bias"],
            "k_b": t[p + "self_attn.k_proj.bias"], "v_b": t[p + "self_attn.v_proj.bias"]})
    got = got.reshape(rows, V)
    for b in range(rows):
        ref = O.decode_first_token_f64(model, (token + 7 * b) % V)["logits"]
        rel = float(np.abs(got[b] - ref).max() / np.abs(ref).max())
        print(f"  row {b} logits max rel {rel:.3g}", flush=True)
        assert rel <= 1e-3
