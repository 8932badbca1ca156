"""VMPrograms for the benchmark configurations, built the way the lowering emits
them for the equivalent JAX programs (tensor instructions through ``graph``).

* ``mlp_c1``: config 1, the f32 two-layer MLP forward
  ``relu(x @ W1 + b1) @ W2 + b2`` (the reference's workload-coverage MLP,
  tools/bench_workloads.py), bias adds and relu folded into the matmul store
  (lowering.py:2486-2601).
* ``gpt_c5``: config 5, a GPT-style pre-LN decoder (learned token and position
  embeddings, fused-QKV attention, tanh-GELU MLP, untied LM head) that prefills
  a prompt and then runs greedy decoding inside one counted loop (``OP_FOR``,
  lowering.py:935-996).  Matmul operands are bf16 with f32 accumulation; the
  residual stream and the layernorm parameters are f32; the KV cache is bf16.

Weights are program inputs, as jax.jit passes a model's parameters (so they
are zero-copy ports, not constants).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

from . import graph as G
from . import vmprogram as V


# ---- config 1 ------------------------------------------------------------------------

def mlp_c1(batch=256, d_in=128, d_hidden=512, d_out=64):
    """Program and input order (x, W1, b1, W2, b2) of the config-1 MLP."""
    g = G.Graph()
    x = g.input((batch, d_in))
    w1, b1 = g.input((d_in, d_hidden)), g.input((d_hidden,))
    w2, b2 = g.input((d_hidden, d_out)), g.input((d_out,))
    # bias per column, then relu as max(h, 0) against the epilogue's constant
    # operand (src 3), in the matmul's store: no phase of its own
    h = g.dot(x, w1, epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_MAX, 3, 0.0, 0.0)], residual=b1)
    y = g.dot(h, w2, epilogue=[(V.SUB_ADD, 2, 0.0, 0.0)], residual=b2)
    g.output(y)
    return g.build()


def mlp_c1_inputs(seed=1001, batch=256, d_in=128, d_hidden=512, d_out=64):
    """BASELINE config 1 draws: x ~ N(0,1), W1 ~ N(0, 1/128), b1 = 0.01,
    W2 ~ N(0, 1/512), b2 = 0."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, d_in), dtype=np.float32)
    w1 = (rng.standard_normal((d_in, d_hidden)) / math.sqrt(d_in)).astype(np.float32)
    b1 = np.full(d_hidden, 0.01, np.float32)
    w2 = (rng.standard_normal((d_hidden, d_out)) / math.sqrt(d_hidden)).astype(np.float32)
    b2 = np.zeros(d_out, np.float32)
    return [x, w1, b1, w2, b2]


# ---- config 5 ------------------------------------------------------------------------

@dataclasses.dataclass(frozen=True)
class GptConfig:
    layers: int = 12
    d: int = 768
    heads: int = 12
    mlp: int = 3072
    vocab: int = 32000
    prompt: int = 512
    steps: int = 128
    eps: float = 1e-5

    @property
    def ctx(self) -> int:            # KV-cache capacity: prompt + decoded tokens
        return self.prompt + self.steps

    @property
    def hd(self) -> int:
        return self.d // self.heads


C5 = GptConfig()

# per-layer parameter names, in input order
LAYER_PARAMS = ("ln1_g", "ln1_b", "w_qkv", "b_qkv", "w_o", "b_o", "ln2_g", "ln2_b", "w_fc", "b_fc",
                "w_proj", "b_proj")


def gpt_param_shapes(c: GptConfig):
    """[(name, shape, dtype)] in program input order (after the prompt ids)."""
    out = [("wte", (c.vocab, c.d), "bf16"), ("wpe", (c.ctx, c.d), "bf16")]
    per = {"ln1_g": ((c.d,), "f32"), "ln1_b": ((c.d,), "f32"), "w_qkv": ((c.d, 3 * c.d), "bf16"),
           "b_qkv": ((3 * c.d,), "f32"), "w_o": ((c.d, c.d), "bf16"), "b_o": ((c.d,), "f32"),
           "ln2_g": ((c.d,), "f32"), "ln2_b": ((c.d,), "f32"), "w_fc": ((c.d, c.mlp), "bf16"),
           "b_fc": ((c.mlp,), "f32"), "w_proj": ((c.mlp, c.d), "bf16"), "b_proj": ((c.d,), "f32")}
    for l in range(c.layers):
        for name in LAYER_PARAMS:
            shape, dt = per[name]
            out.append((f"h{l}.{name}", shape, dt))
    out += [("lnf_g", (c.d,), "f32"), ("lnf_b", (c.d,), "f32"), ("lm_head", (c.d, c.vocab), "bf16")]
    return out


def gpt_inputs(c: GptConfig = C5, seed=1005):
    """BASELINE config 5 draws: every parameter ~ N(0, 0.02) (layernorm gains 1,
    biases 0), prompt ids ~ U[0, vocab).  bf16 parameters are returned as their
    bf16 bit patterns (uint16)."""
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, c.vocab, c.prompt).astype(np.int32)
    arrays = [ids]
    for name, shape, dt in gpt_param_shapes(c):
        base = name.split(".")[-1]
        if base.endswith("_g"):
            a = np.ones(shape, np.float32)
        elif base.startswith("b_") or base.endswith("_b"):
            a = np.zeros(shape, np.float32)
        else:
            a = (rng.standard_normal(shape, dtype=np.float32) * 0.02).astype(np.float32)
        arrays.append(V.f32_to_bf16(a) if dt == "bf16" else a)
    return arrays


def gpt_c5(c: GptConfig = C5, emit_logits: bool = False, trips: int | None = None):
    """Prefill + greedy decode program.  Outputs: the first generated token [1]
    (argmax after the prompt), the ``steps`` tokens decoded after it [steps], and
    with ``emit_logits`` the f32 logits of every step [steps + 1, vocab].
    ``trips`` runs only that many decode steps (same inputs and outputs; for
    separating prefill from decode time)."""
    g = G.Graph()
    H, hd, T, D = c.heads, c.hd, c.prompt, c.d
    C = -(-c.ctx // 8) * 8        # cache capacity: whole 16-byte runs of keys
    ids = g.input((T,), "i32")
    P = {}
    for name, shape, dt in gpt_param_shapes(c):
        P[name] = g.input(shape, dt)
    zero = g.scalar(0, "i32")
    one = g.scalar(1, "i32")
    scale = 1.0 / math.sqrt(hd)
    # K and V are cached as rows, [H, C, hd]: a decode step reads a key the way
    # it reads a value, 16-byte runs of channels (decode attention's krow form;
    # 1.5-2 % more decode tokens/s than a K^T [H, hd, C] cache)
    cache_k = [g.fill((H, C, hd), 0.0, "bf16") for _ in range(c.layers)]
    cache_v = [g.fill((H, C, hd), 0.0, "bf16") for _ in range(c.layers)]
    logits_all = g.fill((c.steps + 1, c.vocab), 0.0) if emit_logits else None

    def mlp_block(x, l, rows):
        h2 = g.layernorm(x, P[f"h{l}.ln2_g"], P[f"h{l}.ln2_b"], c.eps, out_dtype="bf16")
        f = g.dot(h2, P[f"h{l}.w_fc"], out_dtype="bf16", residual=P[f"h{l}.b_fc"],
                  epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_GELU, 0, 0.0, 0.0)])
        xb = g.add(x, g.broadcast_view(P[f"h{l}.b_proj"], (rows, D), (1,)))
        return g.dot(f, P[f"h{l}.w_proj"], residual=xb, epilogue=[(V.SUB_ADD, 1, 0.0, 0.0)])

    def head(x_last, step_idx):
        """final layernorm + LM head on one row -> (token [1], logits [1, vocab])."""
        hf = g.layernorm(x_last, P["lnf_g"], P["lnf_b"], c.eps, out_dtype="bf16")
        logits = g.dot(hf, P["lm_head"])
        _, tok = g.argmax_last(logits)
        if emit_logits:
            g.dynamic_update_slice(logits_all, logits, [step_idx, zero])
        return tok

    # ---- prefill: the whole prompt, causal flash attention, fills the KV cache
    x = g.add(g.convert(g.take_rows(P["wte"], ids), "f32"),
              g.convert(g.slice(P["wpe"], (0, 0), (T, D)), "f32"))
    for l in range(c.layers):
        h = g.layernorm(x, P[f"h{l}.ln1_g"], P[f"h{l}.ln1_b"], c.eps, out_dtype="bf16")
        qkv = g.dot(h, P[f"h{l}.w_qkv"], out_dtype="bf16", residual=P[f"h{l}.b_qkv"],
                    epilogue=[(V.SUB_ADD, 2, 0.0, 0.0)])
        q, k, v = (g.materialize(g.view(qkv, (H, T, hd), (hd, 3 * D, 1), s * D)) for s in range(3))
        g.dynamic_update_slice(cache_k[l], k, [zero, zero, zero])
        g.dynamic_update_slice(cache_v[l], v, [zero, zero, zero])
        att = g.flash_attention(q, k, v, scale, True)                       # [H, T, hd] bf16
        att_rows = g.reshape(g.transpose_view(att, (1, 0, 2)), (T, D))    # [T, H*hd]
        xb = g.add(x, g.broadcast_view(P[f"h{l}.b_o"], (T, D), (1,)))
        x = g.dot(att_rows, P[f"h{l}.w_o"], residual=xb, epilogue=[(V.SUB_ADD, 1, 0.0, 0.0)])
        x = mlp_block(x, l, T)
    tok = head(g.slice(x, (T - 1, 0), (T, D)), zero)                         # [1] i32
    first = g.fill((1,), 0, "i32")
    g.copy_into(first, tok)

    # ---- greedy decode: one token per trip; carries the token and its position
    cur = g.fill((1,), 0, "i32")
    g.copy_into(cur, tok)
    pos = g.fill((), T, "i32")
    out = g.fill((c.steps,), 0, "i32")

    g.begin()
    # both embedding rows are gathered in one phase, converted and added in the next
    tok_row = g.take_rows(P["wte"], cur)
    pos_row = g.dynamic_slice(P["wpe"], [pos, zero], [1, D])
    step = g.add(pos, g.scalar(-T, "i32"))               # this trip's output slot
    x = g.add(g.convert(tok_row, "f32"), g.convert(pos_row, "f32"))
    for l in range(c.layers):
        h = g.layernorm(x, P[f"h{l}.ln1_g"], P[f"h{l}.ln1_b"], c.eps, out_dtype="bf16")
        qkv = g.dot(h, P[f"h{l}.w_qkv"], out_dtype="bf16", residual=P[f"h{l}.b_qkv"],
                    epilogue=[(V.SUB_ADD, 2, 0.0, 0.0)])
        # q, k, v are contiguous thirds of the one row: aliases, not copies
        q, k, v = (g.alias(qkv, s * D, (H, hd)) for s in range(3))
        xb = g.add(x, g.reshape(P[f"h{l}.b_o"], (1, D)))      # beside the QKV matmul
        # attention over the cache prefix [0, pos) and this step's own k, v; the
        # cache takes k, v afterwards, beside the output projection
        att = g.decode_attention(q, k, v, cache_k[l], cache_v[l], pos, scale, krow=True)  # [H, hd] bf16
        g.dynamic_update_slice(cache_k[l], g.reshape(k, (H, 1, hd)), [zero, pos, zero])
        g.dynamic_update_slice(cache_v[l], g.reshape(v, (H, 1, hd)), [zero, pos, zero])
        x = g.dot(g.reshape(att, (1, D)), P[f"h{l}.w_o"], residual=xb,
                  epilogue=[(V.SUB_ADD, 1, 0.0, 0.0)])
        x = mlp_block(x, l, 1)
    nxt = head(x, g.add(step, one))
    # the slot comes from `step`, not `pos`, so that the position moves on in
    # the same phase
    g.dynamic_update_slice(out, nxt, [step])
    g.copy_into(cur, nxt)
    g.copy_into(pos, g.add(pos, one))
    body = g.end()
    g.for_loop(c.steps if trips is None else trips, body)
    g.output(first, out)
    if emit_logits:
        g.output(logits_all)
    return g.build()


def gpt_reference(c: GptConfig, arrays, steps=None, bf16_stores=True):
    """Independent numpy statement of the same decoder (float64 math with bf16
    rounding where the program stores bf16; with ``bf16_stores`` False, no
    rounding: the f32-widened decoder), for pinning the oracle on tiny
    configurations: returns (tokens [1 + steps], logits [1 + steps, vocab])."""
    steps = c.steps if steps is None else steps
    if bf16_stores:
        bf = lambda a: V.bf16_to_f32(V.f32_to_bf16(np.asarray(a, np.float32))).astype(np.float64)
    else:
        bf = lambda a: np.asarray(a, np.float64)
    names = ["ids"] + [n for n, _, _ in gpt_param_shapes(c)]
    P = {}
    for n, a in zip(names, arrays):
        P[n] = a if n == "ids" else (V.bf16_to_f32(a).astype(np.float64) if a.dtype == np.uint16
                                      else a.astype(np.float64))
    H, hd, D = c.heads, c.hd, c.d

    def ln(x, gname, bname):
        mu = x.mean(-1, keepdims=True)
        var = ((x - mu) ** 2).mean(-1, keepdims=True)
        return (x - mu) / np.sqrt(var + c.eps) * P[gname] + P[bname]

    def gelu(x):
        return 0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))

    Kc = np.zeros((c.layers, H, c.ctx, hd))
    Vc = np.zeros((c.layers, H, c.ctx, hd))

    def block(x, l, positions):
        n = x.shape[0]
        h = bf(ln(x, f"h{l}.ln1_g", f"h{l}.ln1_b"))
        qkv = bf(h @ P[f"h{l}.w_qkv"] + P[f"h{l}.b_qkv"])
        q = qkv[:, :D].reshape(n, H, hd).transpose(1, 0, 2)
        k = qkv[:, D:2 * D].reshape(n, H, hd).transpose(1, 0, 2)
        v = qkv[:, 2 * D:].reshape(n, H, hd).transpose(1, 0, 2)
        Kc[l][:, positions] = k
        Vc[l][:, positions] = v
        last = positions[-1]
        s = q @ Kc[l][:, :last + 1].transpose(0, 2, 1) / math.sqrt(hd)
        s = np.where(np.arange(last + 1)[None, None, :] > np.asarray(positions)[None, :, None], -np.inf, s)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        att = bf(p @ Vc[l][:, :last + 1]).transpose(1, 0, 2).reshape(n, D)
        x = x + P[f"h{l}.b_o"] + att @ P[f"h{l}.w_o"]
        h2 = bf(ln(x, f"h{l}.ln2_g", f"h{l}.ln2_b"))
        f = bf(gelu(h2 @ P[f"h{l}.w_fc"] + P[f"h{l}.b_fc"]))
        return x + P[f"h{l}.b_proj"] + f @ P[f"h{l}.w_proj"]

    def logits_of(xrow):
        return bf(ln(xrow, "lnf_g", "lnf_b")) @ P["lm_head"]

    T = c.prompt
    x = P["wte"][P["ids"]] + P["wpe"][:T]
    for l in range(c.layers):
        x = block(x, l, list(range(T)))
    lg = [logits_of(x[T - 1:T])[0]]
    toks = [int(np.argmax(lg[0]))]
    for i in range(steps):
        p = T + i
        x = P["wte"][[toks[-1]]] + P["wpe"][[p]]
        for l in range(c.layers):
            x = block(x, l, [p])
        lg.append(logits_of(x)[0])
        toks.append(int(np.argmax(lg[-1])))
    return np.array(toks, np.int64), np.stack(lg)
