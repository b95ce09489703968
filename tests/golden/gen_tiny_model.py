"""Writes a tiny quantised model directory with the reference's OWN writer
(oracle/_ref/libref.so: llm::QuantWriter, src/quant.cpp:96-134) and checks
that the reference's own loader accepts it (llm::QuantModel::load,
src/quant.cpp:198-238).  Run in the build container only:

    make -C oracle ref && python tests/golden/gen_tiny_model.py

Output: tests/golden/tiny_model/
    config.json                 Qwen2-style config (2 layers, hidden 128,
                                intermediate 320 = 2.5 groups, vocab 160)
    model.q8.llmq, model.q4.llmq  tensors in tools/quantize.cpp:56-73 order
    manifest.json               per file: the tensors in write order with
                                dtype, shape and FNV-1a-64 of each payload
                                (q / scales / zeros, or the bf16 data)
Weights are seeded N(0, 0.05) -> bf16, quantised by the reference.
"""
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)
from oracle.oracle import f32_to_bf16  # noqa: E402
from gen_golden import p, ref_lib, ref_quantize  # noqa: E402

OUT = os.path.join(HERE, "tiny_model")
CONFIG = {
    "architectures": ["Qwen2ForCausalLM"],
    "hidden_size": 128,
    "intermediate_size": 320,
    "num_attention_heads": 2,
    "num_key_value_heads": 1,
    "num_hidden_layers": 2,
    "vocab_size": 160,
    "rope_theta": 1000000.0,
    "rms_norm_eps": 1e-06,
    "tie_word_embeddings": False,
}


def fnv1a64(b):
    h = 0xCBF29CE484222325
    for x in bytes(b):
        h ^= x
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return "%016x" % h


def tiny_entries():
    """The tiny model's bf16 tensors, in tools/quantize.cpp:56-73 order:
    [("m" matrix | "v" vector, name, bf16 bits array)] (seeded; the same
    arrays every call)."""
    H, I, V = CONFIG["hidden_size"], CONFIG["intermediate_size"], CONFIG["vocab_size"]
    hd = H // CONFIG["num_attention_heads"]
    q_out, kv_out = CONFIG["num_attention_heads"] * hd, CONFIG["num_key_value_heads"] * hd
    rng = np.random.default_rng(2024)

    def mat(r, c):
        return f32_to_bf16(rng.standard_normal((r, c), dtype=np.float32) * np.float32(0.05))

    def vec(n, base=0.0):
        return f32_to_bf16(base + rng.standard_normal(n, dtype=np.float32) * np.float32(0.1))

    # tools/quantize.cpp:56-73 order: embed, lm_head, final norm, then per layer
    # q, k, v, o, gate, up, down, input_ln, post_attn_ln, q/k/v bias
    entries = [("m", "model.embed_tokens.weight", mat(V, H)), ("m", "lm_head.weight", mat(V, H)),
               ("v", "model.norm.weight", vec(H, 1.0))]
    for i in range(CONFIG["num_hidden_layers"]):
        pre = f"model.layers.{i}."
        entries += [("m", pre + "self_attn.q_proj.weight", mat(q_out, H)),
                    ("m", pre + "self_attn.k_proj.weight", mat(kv_out, H)),
                    ("m", pre + "self_attn.v_proj.weight", mat(kv_out, H)),
                    ("m", pre + "self_attn.o_proj.weight", mat(H, q_out)),
                    ("m", pre + "mlp.gate_proj.weight", mat(I, H)),
                    ("m", pre + "mlp.up_proj.weight", mat(I, H)),
                    ("m", pre + "mlp.down_proj.weight", mat(H, I)),
                    ("v", pre + "input_layernorm.weight", vec(H, 1.0)),
                    ("v", pre + "post_attention_layernorm.weight", vec(H, 1.0)),
                    ("v", pre + "self_attn.q_proj.bias", vec(q_out)),
                    ("v", pre + "self_attn.k_proj.bias", vec(kv_out)),
                    ("v", pre + "self_attn.v_proj.bias", vec(kv_out))]

    return entries


def main():
    L = ref_lib()
    P = ctypes.c_void_p
    L.ref_writer_new.restype = P
    L.ref_writer_free.argtypes = [P]
    L.ref_writer_add.argtypes = [P, ctypes.c_char_p, P, P, P, ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    L.ref_writer_add.restype = ctypes.c_int
    L.ref_writer_add_bf16.argtypes = [P, ctypes.c_char_p, P, ctypes.c_int64]
    L.ref_writer_add_bf16.restype = ctypes.c_int
    L.ref_writer_write.argtypes = [P, ctypes.c_char_p]
    L.ref_writer_write.restype = ctypes.c_int
    L.ref_quantmodel_layers.argtypes = [ctypes.c_char_p, ctypes.c_int]
    L.ref_quantmodel_layers.restype = ctypes.c_int

    os.makedirs(OUT, exist_ok=True)
    with open(os.path.join(OUT, "config.json"), "w") as f:
        json.dump(CONFIG, f, indent=2)
    H, I, V = CONFIG["hidden_size"], CONFIG["intermediate_size"], CONFIG["vocab_size"]
    hd = H // CONFIG["num_attention_heads"]
    q_out, kv_out = CONFIG["num_attention_heads"] * hd, CONFIG["num_key_value_heads"] * hd

    entries = tiny_entries()

    manifest = {}
    for kind, fname in ((0, "model.q8.llmq"), (1, "model.q4.llmq")):
        h = L.ref_writer_new()
        items = []
        for typ, name, arr in entries:
            if typ == "v":
                assert L.ref_writer_add_bf16(h, name.encode(), p(arr), arr.size) == 0
                items.append({"name": name, "dtype": "bf16", "shape": [int(arr.size)],
                              "data": fnv1a64(arr.tobytes())})
            else:
                q, s, z, _ = ref_quantize(L, arr, kind)
                rows, cols = arr.shape
                assert L.ref_writer_add(h, name.encode(), p(q), p(s), p(z), kind, rows, cols) == 0
                it = {"name": name, "dtype": "int4" if kind else "int8", "shape": [rows, cols],
                      "q": fnv1a64(q.tobytes()), "scales": fnv1a64(s.tobytes())}
                if kind == 1:
                    it["zeros"] = fnv1a64(z.tobytes())
                items.append(it)
        assert L.ref_writer_write(h, os.path.join(OUT, fname).encode()) == 0
        L.ref_writer_free(h)
        n = L.ref_quantmodel_layers(OUT.encode(), kind)
        assert n == CONFIG["num_hidden_layers"], n
        manifest[fname] = items
    with open(os.path.join(OUT, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print("wrote", OUT, {k: len(v) for k, v in manifest.items()})


if __name__ == "__main__":
    main()
