"""Stage programs of dependent 1-row GEMVs (include/iq.h, iq_chain_*), and
the decode step built from them.

DecodeStep is the quantised part of the reference's decode step,
GpuBatch::Impl::launch_sequence (kernels/batch_gpu.cu:186-215), for B
sequences (B = 1..32, GpuBatch::kMaxRows, kernels/batch_gpu.h:80) of one
token each at position 0: the quantised embedding gather of the B tokens
(launch_embedding_q), then per layer, for each of the B rows

    q|k|v  = rmsnorm(h, input_ln) . W_qkv^T + b_qkv          (one stage)
    h'     = h + attn . W_o^T                                  (one stage)
    act    = silu(n . W_gate^T) * (n . W_up^T),
             n = rmsnorm(h', post_attn_ln)                    (one stage)
    h''    = h' + act . W_down^T                               (one stage)

and logits = rmsnorm(h, final_norm) . W_head^T.  At position 0 the
attention over the single cached key has softmax weight 1, so attn is the
value row of each query head's key/value head (IQ_IN_GQA); RoPE changes q
and k only.  Every intermediate vector has its own buffer (static
single-assignment), so all of them can be inspected after a step.
"""
import ctypes

import torch

from . import ops

IN_PLAIN, IN_RMSNORM, IN_GQA = 0, 1, 2
OUT_STORE, OUT_RESIDUAL, OUT_SWIGLU = 0, 1, 2


IqStage = ops.IqStage


def _lib():
    return ops.lib()


def _p(t):
    return None if t is None else t.data_ptr()


class Stage:
    """One stage: y_i = out_op(dequant(Ws[i]) . in_op(x) + biases[i])."""

    def __init__(self, Ws, x, ys, in_op=IN_PLAIN, out_op=OUT_STORE, biases=None, norm=None, eps=0.0,
                 residual=None, gqa=(0, 0), rows=1):
        self.Ws, self.x, self.ys = list(Ws), x, list(ys)
        self.rows = rows
        self.in_op, self.out_op = in_op, out_op
        self.biases = list(biases) if biases is not None else [None] * len(self.Ws)
        self.norm, self.eps, self.residual, self.gqa = norm, eps, residual, gqa

    def to_c(self):
        s = IqStage()
        s.in_op, s.out_op, s.n = self.in_op, self.out_op, len(self.Ws)
        s.gqa_head_dim, s.gqa_group = self.gqa
        s.eps = self.eps
        s.rows = self.rows
        s.x, s.norm, s.residual = _p(self.x), _p(self.norm), _p(self.residual)
        for i, W in enumerate(self.Ws):
            s.W[i] = W._c
            s.bias[i] = _p(self.biases[i])
        for i, y in enumerate(self.ys):
            s.y[i] = _p(y)
        return s


class Chain:
    """A validated program on the current device (iq_chain_create)."""

    def __init__(self, stages):
        self.stages = list(stages)  # keeps the tensors alive
        arr = (IqStage * len(self.stages))(*[s.to_c() for s in self.stages])
        h = ctypes.c_void_p()
        rc = _lib().iq_chain_create(arr, len(self.stages), ctypes.byref(h))
        ops._check(rc, "iq_chain_create")
        self._h = h

    def run(self, stream=None):
        ops._check(_lib().iq_chain_run(self._h, ops._stream(stream)), "iq_chain_run")

    def close(self):
        if getattr(self, "_h", None):
            _lib().iq_chain_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Arena:
    """fp32 vectors carved from one device tensor, each starting on its own
    1 KiB boundary (no two vectors share a cache line)."""

    def __init__(self, sizes, device="cuda"):
        pad = [(n + 255) // 256 * 256 for n in sizes]
        self.buf = torch.zeros(sum(pad) + 256, dtype=torch.float32, device=device)
        base = (-(self.buf.data_ptr() // 4)) % 256
        self.views, off = [], base
        for n, p in zip(sizes, pad):
            self.views.append(self.buf[off:off + n])
            off += p


class DecodeStep:
    """The quantised decode step of one token at position 0 (module
    docstring).  `model` has: cfg dict (hidden, inter, heads, kv_heads,
    head_dim, vocab, layers, eps), embed / head (QuantView), final_norm
    (bf16 int16 tensor), layers: list of dicts with QuantViews q, k, v, o,
    gate, up, down, bf16 tensors input_ln, post_ln and optional q_b, k_b, v_b.
    rows: B sequences; every vector below is [B][n] row-major."""

    def __init__(self, model, device="cuda", rows=1):
        c = model["cfg"]
        H, I, V = c["hidden"], c["inter"], c["vocab"]
        nh, nkv, hd, L = c["heads"], c["kv_heads"], c["head_dim"], c["layers"]
        qo, kvo = nh * hd, nkv * hd
        B = self.rows = int(rows)
        sizes = [H]
        for _ in range(L):
            sizes += [qo, kvo, kvo, H, I, H]
        sizes += [V]
        self.arena = Arena([B * n for n in sizes], device)
        vs = iter(self.arena.views)
        self.h0 = next(vs)
        self.ids = torch.zeros(B, dtype=torch.int64, device=device)
        self.model = model
        self.per_layer = []
        stages = []
        h = self.h0
        for li in range(L):
            Lw = model["layers"][li]
            q, k, v, h1, act, h2 = (next(vs) for _ in range(6))
            stages.append(Stage([Lw["q"], Lw["k"], Lw["v"]], h, [q, k, v], IN_RMSNORM, OUT_STORE,
                                biases=[Lw.get("q_b"), Lw.get("k_b"), Lw.get("v_b")], norm=Lw["input_ln"],
                                eps=c["eps"], rows=B))
            stages.append(Stage([Lw["o"]], v, [h1], IN_GQA, OUT_RESIDUAL, residual=h, gqa=(hd, nh // nkv), rows=B))
            stages.append(Stage([Lw["gate"], Lw["up"]], h1, [act], IN_RMSNORM, OUT_SWIGLU, norm=Lw["post_ln"],
                                eps=c["eps"], rows=B))
            stages.append(Stage([Lw["down"]], act, [h2], IN_PLAIN, OUT_RESIDUAL, residual=h1, rows=B))
            self.per_layer.append(dict(h=h, q=q, k=k, v=v, h1=h1, act=act, h2=h2))
            h = h2
        self.logits = next(vs)
        stages.append(Stage([model["head"]], h, [self.logits], IN_RMSNORM, OUT_STORE, norm=model["final_norm"],
                            eps=c["eps"], rows=B))
        self.h_last = h
        self.chain = Chain(stages)

    def step(self, token_id=None, stream=None):
        """Embedding gather of the B token ids `token_id` (an int for every
        row, or a sequence of B ints; None: the ids already in self.ids),
        then the chain.  Asynchronous on the stream."""
        if token_id is not None:
            if isinstance(token_id, int):
                self.ids.fill_(int(token_id))
            else:
                self.ids.copy_(torch.tensor([int(t) for t in token_id], dtype=torch.int64))
        H = self.model["cfg"]["hidden"]
        ops.launch_embedding_q(self.model["embed"], self.ids, self.rows, H, self.h0, stream)
        self.chain.run(stream)

    def weight_bytes(self):
        n = self.rows * (self.model["embed"].nbytes() // self.model["embed"].rows)  # the gathered rows
        for Lw in self.model["layers"]:
            n += sum(Lw[k].nbytes() for k in ("q", "k", "v", "o", "gate", "up", "down"))
        return n + self.model["head"].nbytes()
