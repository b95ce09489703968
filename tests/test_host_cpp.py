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
