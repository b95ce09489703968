"""The decode-step chain (include/iq.h iq_chain_*, infer_amd/chain.py)
against the oracle's float64 forward of one token at position 0
(oracle.decode_first_token_f64, src/forward.cpp:160-262 on dequantised
weights), through the C ABI.

Per stage, each output is checked against the oracle applied to the chain's
own input vectors (every intermediate has its own buffer): the GEMV
conditioning tolerance of tests/test_ops_gpu.cu:199-206 (5e-6 of sum |w x|),
propagated through the SwiGLU and residual epilogues.  End to end, the
logits are within max|err| / max|ref| <= 1e-3 of the float64 forward
(the tolerance stated for the decode path).  Also: determinism over runs, a 7B-shaped
chain (28 layers, int4 layers, int8 head) checked stage by stage on
sampled rows, and the host's overlap check (IQ_EALIAS)."""
import ctypes

import numpy as np
import pytest
import torch

from infer_amd import chain as C
from infer_amd import ops
from oracle import oracle as O
from tests.gpu_util import KGEMV_TOL, say

pytestmark = pytest.mark.gpu


def bf16_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda()


class Mat:
    """A packed matrix on the device with its host codes (seeded bf16
    weights quantised by the oracle, or random codes for big shapes)."""

    def __init__(self, rng, rows, cols, kind, quantize=True, sd=0.02):
        self.kind, self.rows, self.cols = kind, rows, cols
        G = O.groups(cols)
        if quantize:
            w = O.seeded_bf16(rng, (rows, cols), sd)
            self.q, self.s, self.z = O.quantize(w, kind)
        else:
            nq = rows * cols // 2 if kind == 1 else rows * cols
            if kind == 1:
                self.q = rng.integers(0, 256, nq, dtype=np.uint8)
                self.z = rng.integers(0, 16, (rows, G), dtype=np.uint8)
            else:
                self.q = rng.integers(-127, 128, nq, dtype=np.int16).astype(np.int8).view(np.uint8)
                self.z = None
            self.s = O.f32_to_bf16((rng.uniform(2e-4, 8e-4, (rows, G)) * sd / 0.02).astype(np.float32))
        self.view = ops.upload_q(kind, rows, cols, self.q, self.s, self.z)

    def dq(self, idx=None):
        if idx is None:
            idx = np.arange(self.rows)
        rb = self.cols // 2 if self.kind == 1 else self.cols
        q = np.asarray(self.q).reshape(self.rows, rb)[idx]
        z = None if self.z is None else np.asarray(self.z).reshape(self.rows, -1)[idx]
        return O.dequant_matrix(q, np.asarray(self.s).reshape(self.rows, -1)[idx], z, self.kind, len(idx), self.cols)


def make_model(rng, H, I, nh, nkv, hd, V, L, kind, head_kind, quantize=True, bias=True):
    cfg = dict(hidden=H, inter=I, heads=nh, kv_heads=nkv, head_dim=hd, vocab=V, layers=L, eps=1e-6)
    normb = lambda n: O.f32_to_bf16(rng.uniform(0.6, 1.4, n).astype(np.float32))
    host = {"cfg": cfg, "layers": []}
    dev = {"cfg": cfg, "layers": []}
    for _ in range(L):
        hl, dl = {}, {}
        for name, (r, c) in dict(q=(nh * hd, H), k=(nkv * hd, H), v=(nkv * hd, H), o=(H, nh * hd),
                                 gate=(I, H), up=(I, H), down=(H, I)).items():
            m = Mat(rng, r, c, kind, quantize)
            hl[name] = m
            dl[name] = m.view
        for name in ("input_ln", "post_ln"):
            hl[name] = normb(H)
            dl[name] = bf16_dev(hl[name])
        if bias:
            for name, n in (("q_b", nh * hd), ("k_b", nkv * hd), ("v_b", nkv * hd)):
                hl[name] = O.seeded_bf16(rng, (n,), 0.3)
                dl[name] = bf16_dev(hl[name])
        host["layers"].append(hl)
        dev["layers"].append(dl)
    host["embed"] = Mat(rng, V, H, head_kind, quantize, sd=0.5)
    host["head"] = Mat(rng, V, H, head_kind, quantize)
    host["final_norm"] = normb(H)
    dev["embed"], dev["head"] = host["embed"].view, host["head"].view
    dev["final_norm"] = bf16_dev(host["final_norm"])
    return host, dev


def f64(t):
    return t.detach().cpu().numpy().astype(np.float64)


def check_gemv(got, W, x, idx, what, bias=None, slack=None):
    """|got - W.x (+b)| <= 5e-6 sum |w x| (+ slack: the fp32 rounding of a
    residual sum) on rows idx; returns the reference and its conditioning."""
    dq = W.dq(idx).astype(np.float64)
    ref = dq @ x
    cond = np.abs(dq) @ np.abs(x)
    if bias is not None:
        b = O.bf16_to_f32(bias[idx]).astype(np.float64)
        ref, cond = ref + b, cond + np.abs(b)
    err = np.abs(got[idx] - ref)
    if slack is not None:
        err = np.maximum(err - slack[idx], 0.0)
    worst = float((err / np.maximum(cond, 1e-30)).max())
    assert worst <= KGEMV_TOL, f"{what}: conditioning error {worst:.3g}"
    return ref, cond


def check_step(step, host, idx_of=None, layers=None):
    """Every stage's output against the oracle on the chain's own inputs."""
    c = host["cfg"]
    eps = c["eps"]
    sel = (lambda n: np.arange(n)) if idx_of is None else idx_of
    L = len(step.per_layer)
    for li in (range(L) if layers is None else layers):
        b, hl = step.per_layer[li], host["layers"][li]
        h = f64(b["h"])
        n = O.rmsnorm_f64(h, hl["input_ln"], eps)
        for name in ("q", "k", "v"):
            check_gemv(f64(b[name]), hl[name], n, sel(hl[name].rows), f"L{li}.{name}", hl.get(name + "_b"))
        ctx = O.attention_single_key(f64(b["v"]), c["heads"], c["kv_heads"], c["head_dim"])
        idx = sel(c["hidden"])
        h1 = f64(b["h1"])
        check_gemv(h1 - h, hl["o"], ctx, idx, f"L{li}.o+res", slack=np.abs(h1) * 2.0 ** -24)
        n2 = O.rmsnorm_f64(f64(b["h1"]), hl["post_ln"], eps)
        idx = sel(c["inter"])
        dg, du = hl["gate"].dq(idx).astype(np.float64), hl["up"].dq(idx).astype(np.float64)
        g, u = dg @ n2, du @ n2
        cg, cu = np.abs(dg) @ np.abs(n2), np.abs(du) @ np.abs(n2)
        act_ref = O.silu_f64(g) * u
        bound = 2 * KGEMV_TOL * (1.1 * cg * np.abs(u) + cu * np.abs(O.silu_f64(g))) + 1e-6 * np.abs(act_ref) + 1e-30
        err = np.abs(f64(b["act"])[idx] - act_ref)
        assert np.all(err <= bound), f"L{li}.swiglu: worst {float((err / bound).max()):.3g} of the bound"
        idx = sel(c["hidden"])
        h2 = f64(b["h2"])
        check_gemv(h2 - h1, hl["down"], f64(b["act"]), idx, f"L{li}.down+res", slack=np.abs(h2) * 2.0 ** -24)
    nf = O.rmsnorm_f64(f64(step.h_last), host["final_norm"], eps)
    check_gemv(f64(step.logits), host["head"], nf, sel(host["head"].rows), "lm_head")


def oracle_model(host):
    c = host["cfg"]
    m = {"cfg": c, "embed_dq": host["embed"].dq(), "head_dq": host["head"].dq(),
         "final_norm": host["final_norm"], "layers": []}
    for hl in host["layers"]:
        d = {k: hl[k].dq() for k in ("q", "k", "v", "o", "gate", "up", "down")}
        d.update({k: hl.get(k) for k in ("input_ln", "post_ln", "q_b", "k_b", "v_b")})
        m["layers"].append(d)
    return m


@pytest.mark.parametrize("kind,head_kind", [(1, 0), (0, 0), (1, 1)])
def test_chain_small_model_matches_forward(kind, head_kind):
    rng = np.random.default_rng(10 + 3 * kind + head_kind)
    host, dev = make_model(rng, H=512, I=1536, nh=4, nkv=2, hd=128, V=1000, L=3, kind=kind, head_kind=head_kind)
    say("chain small", kind, head_kind)
    step = C.DecodeStep(dev)
    step.step(7)
    torch.cuda.synchronize()
    check_step(step, host)
    ref = O.decode_first_token_f64(oracle_model(host), 7)
    got = f64(step.logits)
    rel = float(np.abs(got - ref["logits"]).max() / np.abs(ref["logits"]).max())
    say(f"  end-to-end logits max rel {rel:.3g}")
    assert rel <= 1e-3
    # deterministic: a second run writes the same bits
    first = step.logits.clone()
    step.step(7)
    torch.cuda.synchronize()
    assert torch.equal(first, step.logits)


def test_chain_1p5b_shapes_two_layers():
    """Qwen2.5-1.5B widths (hidden 1536, intermediate 8960: 70 groups, a
    2-group last int4 slice), 12 query / 2 kv heads, int4 + int8 head."""
    rng = np.random.default_rng(15)
    host, dev = make_model(rng, H=1536, I=8960, nh=12, nkv=2, hd=128, V=4096, L=2, kind=1, head_kind=0,
                           quantize=False)
    say("chain 1.5B shapes")
    step = C.DecodeStep(dev)
    step.step(11)
    torch.cuda.synchronize()
    pick = np.random.default_rng(0)
    check_step(step, host, idx_of=lambda n: np.unique(np.r_[0, 15, n - 1, pick.choice(n, 96)]))


def test_chain_7b_shapes_sampled():
    """The benchmark's program: Qwen2.5-7B widths, 28 layers int4 and the
    int8 lm_head 152064 x 3584, checked stage by stage on sampled rows."""
    rng = np.random.default_rng(7)
    host, dev = make_model(rng, H=3584, I=18944, nh=28, nkv=4, hd=128, V=152064, L=28, kind=1, head_kind=0,
                           quantize=False)
    say("chain 7B shapes")
    step = C.DecodeStep(dev)
    step.step(1234)
    torch.cuda.synchronize()
    logits = f64(step.logits)
    assert np.all(np.isfinite(logits))
    pick = np.random.default_rng(1)
    check_step(step, host, idx_of=lambda n: np.unique(np.r_[0, n - 1, pick.choice(n, 48)]), layers=[0, 1, 13, 27])


def test_chain_rejects_in_place_stages():
    """A stage whose output overlaps its own input (or residual) is refused
    with IQ_EALIAS; a later stage may reuse an earlier stage's buffers."""
    rng = np.random.default_rng(3)
    W = Mat(rng, 256, 256, 1)
    x = torch.zeros(256, device="cuda")
    y = torch.zeros(256, device="cuda")
    with pytest.raises(RuntimeError, match="overlaps"):
        C.Chain([C.Stage([W.view], x, [x])])
    with pytest.raises(RuntimeError, match="overlaps"):
        C.Chain([C.Stage([W.view], x, [y], out_op=C.OUT_RESIDUAL, residual=y)])
    C.Chain([C.Stage([W.view], x, [y]), C.Stage([W.view], y, [x])]).close()


class RowView:
    """Row b of a B-row DecodeStep, shaped like a 1-row step for check_step."""

    def __init__(self, step, b):
        B = step.rows
        row = lambda t: t.view(B, -1)[b]
        self.per_layer = [{k: row(v) for k, v in d.items()} for d in step.per_layer]
        self.h_last = row(step.h_last)
        self.logits = row(step.logits)


@pytest.mark.parametrize("B", [2, 3, 4, 6, 16, 32])
@pytest.mark.parametrize("kind,head_kind", [(1, 0), (0, 0)])
def test_chain_rows_small_model_matches_forward(B, kind, head_kind):
    """B sequences of one token each: 2..4 rows on the fused R-row stages
    (one launch per stage), more on the B-row stages (rows GEMV + epilogue;
    at 5..16 rows the narrow ones on operand preparation + gemvh);
    every stage of every row against the oracle on the chain's own inputs,
    and every row's logits against the float64 forward of its token."""
    rng = np.random.default_rng(100 + B + 3 * kind + head_kind)
    host, dev = make_model(rng, H=512, I=1536, nh=4, nkv=2, hd=128, V=1000, L=3, kind=kind, head_kind=head_kind)
    tokens = [int(t) for t in rng.integers(0, 1000, B)]
    say("chain rows small", B, kind, head_kind)
    step = C.DecodeStep(dev, rows=B)
    step.step(tokens)
    torch.cuda.synchronize()
    om = oracle_model(host)
    worst = 0.0
    for b in range(B):
        check_step(RowView(step, b), host)
        ref = O.decode_first_token_f64(om, tokens[b])
        got = f64(RowView(step, b).logits)
        worst = max(worst, float(np.abs(got - ref["logits"]).max() / np.abs(ref["logits"]).max()))
    say(f"  end-to-end logits max rel {worst:.3g} over {B} rows")
    assert worst <= 1e-3
    first = step.logits.clone()
    step.step(tokens)
    torch.cuda.synchronize()
    assert torch.equal(first, step.logits)


@pytest.mark.parametrize("B", [2, 3, 4, 16, 32])
def test_chain_rows_7b_shapes_sampled(B):
    """The 7B program (28 int4 layers, int8 lm_head) at B rows: at 2..4 rows
    q|k|v, o, gate|up and (2 rows) the head on fused R-row stages, down
    (K = 18944) and the head at 3..4 rows on the B-row stages (at 2 rows the
    1-row kernel's K-split instance writing the epilogue's range sums); at
    16 / 32 gate|up on the 32-row tile kernel; stage by stage on sampled
    output rows of a few layers and sequences."""
    rng = np.random.default_rng(70 + B)
    host, dev = make_model(rng, H=3584, I=18944, nh=28, nkv=4, hd=128, V=152064, L=28, kind=1, head_kind=0,
                           quantize=False)
    tokens = [int(t) for t in rng.integers(0, 152064, B)]
    say("chain rows 7B", B)
    step = C.DecodeStep(dev, rows=B)
    step.step(tokens)
    torch.cuda.synchronize()
    assert np.all(np.isfinite(f64(step.logits)))
    pick = np.random.default_rng(2)
    for b in (0, B // 2, B - 1):
        check_step(RowView(step, b), host, idx_of=lambda n: np.unique(np.r_[0, n - 1, pick.choice(n, 32)]),
                   layers=[0, 27])


def test_chain_rows_embedding_input_norm():
    """A B-row RMSNorm stage whose input no stage of the chain writes (its
    row sums of squares come from the chain's own pass) and a mixed program:
    a 1-row stage after B-row ones."""
    rng = np.random.default_rng(12)
    B, K, N = 5, 1024, 768
    W = Mat(rng, N, K, 1)
    W1 = Mat(rng, 256, N, 0)
    x = rng.standard_normal((B, K)).astype(np.float32) * 3.0
    nb = O.f32_to_bf16(rng.uniform(0.5, 1.5, K).astype(np.float32))
    xd = torch.from_numpy(x).cuda()
    y = torch.zeros(B * N, device="cuda")
    y1 = torch.zeros(256, device="cuda")
    ch = C.Chain([C.Stage([W.view], xd, [y], C.IN_RMSNORM, C.OUT_STORE, norm=bf16_dev(nb), eps=1e-5, rows=B),
                  C.Stage([W1.view], y, [y1], rows=1)])
    ch.run()
    torch.cuda.synchronize()
    yh = f64(y).reshape(B, N)
    for b in range(B):
        n = O.rmsnorm_f64(x[b], nb, 1e-5)
        check_gemv(yh[b], W, n, np.arange(N), f"row {b}")
    check_gemv(f64(y1), W1, yh[0], np.arange(256), "1-row stage after B-row stages")
    ch.close()
