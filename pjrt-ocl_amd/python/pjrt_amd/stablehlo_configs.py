"""The benchmark configurations as StableHLO module text, in the form JAX
prints a jitted function (``jax.jit(f).lower(...).as_text()``): the input of
the drop-in path, which lowers it (``lowering.lower_text``), schedules it and
runs it.  bench.py times these beside the hand-built programs of ``configs``;
the tests lower them too.

jax is not installed in this image, so the texts are written out following
JAX's lowering rules (jnp.mean = reduce-sum / size, integer_pow by repeated
squaring, jax.nn.softmax = exp(x - max) / sum, einsum = dot_general with
batching dimensions); which exact StableHLO a given JAX version emits is not
pinned here.  Each builder returns the text for the given sizes; its docstring
is the JAX function it stands for."""


def _t(shape, dt="f32"):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def mlp(b=256, d_in=128, h=512, d_out=64):
    """def f(x, w1, b1, w2, b2): return jax.nn.relu(x @ w1 + b1) @ w2 + b2"""
    X, W1, B1, W2, B2 = _t((b, d_in)), _t((d_in, h)), _t((h,)), _t((h, d_out)), _t((d_out,))
    H, Y = _t((b, h)), _t((b, d_out))
    return f"""
module @jit_f attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {X} {{mhlo.layout_mode = "default"}}, %arg1: {W1}, %arg2: {B1}, %arg3: {W2}, %arg4: {B2}) -> ({Y} {{jax.result_info = ""}}) {{
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : ({X}, {W1}) -> {H}
    %1 = stablehlo.broadcast_in_dim %arg2, dims = [1] : ({B1}) -> {H}
    %2 = stablehlo.add %0, %1 : {H}
    %3 = call @relu(%2) : ({H}) -> {H}
    %4 = stablehlo.dot_general %3, %arg3, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : ({H}, {W2}) -> {Y}
    %5 = stablehlo.broadcast_in_dim %arg4, dims = [1] : ({B2}) -> {Y}
    %6 = stablehlo.add %4, %5 : {Y}
    return %6 : {Y}
  }}
  func.func private @relu(%arg0: {H}) -> {H} {{
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.broadcast_in_dim %cst, dims = [] : (tensor<f32>) -> {H}
    %1 = stablehlo.maximum %arg0, %0 : {H}
    return %1 : {H}
  }}
}}
"""


def ln_gelu(rows=64, d=512, out="bf16"):
    """def f(x, g, b):
         mu = jnp.mean(x, -1, keepdims=True)
         var = jnp.mean((x - mu) ** 2, -1, keepdims=True)
         y = (x - mu) * jax.lax.rsqrt(var + 1e-5) * g + b
         return jax.nn.gelu(y, approximate=True).astype(jnp.bfloat16)"""
    X, R, R1, V = _t((rows, d)), _t((rows,)), _t((rows, 1)), _t((d,))
    O = _t((rows, d), out)
    return f"""
module @jit_f {{
  func.func public @main(%arg0: {X}, %arg1: {V}, %arg2: {V}) -> {O} {{
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.add across dimensions = [1] : ({X}, tensor<f32>) -> {R}
    %1 = stablehlo.broadcast_in_dim %0, dims = [0] : ({R}) -> {R1}
    %cst_0 = stablehlo.constant dense<{float(d):.6e}> : tensor<f32>
    %2 = stablehlo.broadcast_in_dim %cst_0, dims = [] : (tensor<f32>) -> {R1}
    %3 = stablehlo.divide %1, %2 : {R1}
    %4 = stablehlo.broadcast_in_dim %3, dims = [0, 1] : ({R1}) -> {X}
    %5 = stablehlo.subtract %arg0, %4 : {X}
    %6 = stablehlo.multiply %5, %5 : {X}
    %7 = stablehlo.reduce(%6 init: %cst) applies stablehlo.add across dimensions = [1] : ({X}, tensor<f32>) -> {R}
    %8 = stablehlo.broadcast_in_dim %7, dims = [0] : ({R}) -> {R1}
    %9 = stablehlo.divide %8, %2 : {R1}
    %cst_1 = stablehlo.constant dense<9.99999974E-6> : tensor<f32>
    %10 = stablehlo.broadcast_in_dim %cst_1, dims = [] : (tensor<f32>) -> {R1}
    %11 = stablehlo.add %9, %10 : {R1}
    %12 = stablehlo.rsqrt %11 : {R1}
    %13 = stablehlo.broadcast_in_dim %12, dims = [0, 1] : ({R1}) -> {X}
    %14 = stablehlo.multiply %5, %13 : {X}
    %15 = stablehlo.broadcast_in_dim %arg1, dims = [1] : ({V}) -> {X}
    %16 = stablehlo.multiply %14, %15 : {X}
    %17 = stablehlo.broadcast_in_dim %arg2, dims = [1] : ({V}) -> {X}
    %18 = stablehlo.add %16, %17 : {X}
    %19 = stablehlo.multiply %18, %18 : {X}
    %20 = stablehlo.multiply %18, %19 : {X}
    %cst_2 = stablehlo.constant dense<4.471500e-02> : tensor<f32>
    %21 = stablehlo.broadcast_in_dim %cst_2, dims = [] : (tensor<f32>) -> {X}
    %22 = stablehlo.multiply %21, %20 : {X}
    %23 = stablehlo.add %18, %22 : {X}
    %cst_3 = stablehlo.constant dense<0.797884583> : tensor<f32>
    %24 = stablehlo.broadcast_in_dim %cst_3, dims = [] : (tensor<f32>) -> {X}
    %25 = stablehlo.multiply %24, %23 : {X}
    %26 = stablehlo.tanh %25 : {X}
    %cst_4 = stablehlo.constant dense<1.000000e+00> : tensor<f32>
    %27 = stablehlo.broadcast_in_dim %cst_4, dims = [] : (tensor<f32>) -> {X}
    %28 = stablehlo.add %27, %26 : {X}
    %cst_5 = stablehlo.constant dense<5.000000e-01> : tensor<f32>
    %29 = stablehlo.broadcast_in_dim %cst_5, dims = [] : (tensor<f32>) -> {X}
    %30 = stablehlo.multiply %29, %28 : {X}
    %31 = stablehlo.multiply %18, %30 : {X}
    %32 = stablehlo.convert %31 : ({X}) -> {O}
    return %32 : {O}
  }}
}}
"""


def matmul(m=256, k=128, n=192, dt="bf16", out="f32"):
    """def f(a, b): return jnp.dot(a, b, preferred_element_type=jnp.float32)"""
    A, B, C = _t((m, k), dt), _t((k, n), dt), _t((m, n), out)
    return f"""
module @jit_f {{
  func.func public @main(%arg0: {A}, %arg1: {B}) -> {C} {{
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : ({A}, {B}) -> {C}
    return %0 : {C}
  }}
}}
"""


def attention(b=1, h=2, t=128, d=64, dt="bf16", causal=True):
    """def f(q, k, v):   # [B, H, T, D]
         s = jnp.einsum("bhqd,bhkd->bhqk", q, k, preferred_element_type=jnp.float32) * d ** -0.5
         s = jnp.where(jnp.tril(jnp.ones((T, T), bool)), s, -jnp.inf)   # when causal
         p = jax.nn.softmax(s, axis=-1).astype(q.dtype)
         return jnp.einsum("bhqk,bhkd->bhqd", p, v, preferred_element_type=jnp.float32).astype(q.dtype)"""
    Q = _t((b, h, t, d), dt)
    S, SB = _t((b, h, t, t)), _t((b, h, t, t), dt)
    R, R1 = _t((b, h, t)), _t((b, h, t, 1))
    O32, O = _t((b, h, t, d)), _t((b, h, t, d), dt)
    M, MB = _t((t, t), "i32"), _t((t, t), "i1")
    scale = d ** -0.5
    mask = f"""
    %m0 = stablehlo.iota dim = 0 : {M}
    %m1 = stablehlo.iota dim = 1 : {M}
    %m2 = stablehlo.compare  GE, %m0, %m1,  SIGNED : ({M}, {M}) -> {MB}
    %m3 = stablehlo.broadcast_in_dim %m2, dims = [2, 3] : ({MB}) -> {_t((b, h, t, t), "i1")}
    %ninf = stablehlo.constant dense<0xFF800000> : tensor<f32>
    %m4 = stablehlo.broadcast_in_dim %ninf, dims = [] : (tensor<f32>) -> {S}
    %s2 = stablehlo.select %m3, %s1, %m4 : {_t((b, h, t, t), "i1")}, {S}""" if causal else """
    %s2 = stablehlo.add %s1, %zero_s : """ + S
    zero = "" if causal else f"""
    %zc = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %zero_s = stablehlo.broadcast_in_dim %zc, dims = [] : (tensor<f32>) -> {S}"""
    return f"""
module @jit_f {{
  func.func public @main(%arg0: {Q}, %arg1: {Q}, %arg2: {Q}) -> {O} {{
    %s0 = stablehlo.dot_general %arg0, %arg1, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [3], precision = [DEFAULT, DEFAULT] : ({Q}, {Q}) -> {S}
    %c = stablehlo.constant dense<{scale:.9e}> : tensor<f32>
    %cb = stablehlo.broadcast_in_dim %c, dims = [] : (tensor<f32>) -> {S}
    %s1 = stablehlo.multiply %s0, %cb : {S}{zero}{mask}
    %mi = stablehlo.constant dense<0xFF800000> : tensor<f32>
    %r0 = stablehlo.reduce(%s2 init: %mi) applies stablehlo.maximum across dimensions = [3] : ({S}, tensor<f32>) -> {R}
    %r1 = stablehlo.broadcast_in_dim %r0, dims = [0, 1, 2] : ({R}) -> {R1}
    %r2 = stablehlo.broadcast_in_dim %r1, dims = [0, 1, 2, 3] : ({R1}) -> {S}
    %e0 = stablehlo.subtract %s2, %r2 : {S}
    %e1 = stablehlo.exponential %e0 : {S}
    %z = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %u0 = stablehlo.reduce(%e1 init: %z) applies stablehlo.add across dimensions = [3] : ({S}, tensor<f32>) -> {R}
    %u1 = stablehlo.broadcast_in_dim %u0, dims = [0, 1, 2] : ({R}) -> {R1}
    %u2 = stablehlo.broadcast_in_dim %u1, dims = [0, 1, 2, 3] : ({R1}) -> {S}
    %p0 = stablehlo.divide %e1, %u2 : {S}
    %p1 = stablehlo.convert %p0 : ({S}) -> {SB}
    %o0 = stablehlo.dot_general %p1, %arg2, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [2], precision = [DEFAULT, DEFAULT] : ({SB}, {Q}) -> {O32}
    %o1 = stablehlo.convert %o0 : ({O32}) -> {O}
    return %o1 : {O}
  }}
}}
"""


# ---- config 5: the GPT decoder as a JAX program ---------------------------------------------

class _Emit:
    """SSA text builder for one function body."""

    def __init__(self, indent="    "):
        self.lines, self.n, self.ind = [], 0, indent

    def new(self, text):
        name = f"%v{self.n}"
        self.n += 1
        self.lines.append(f"{self.ind}{name} = {text}")
        return name

    def const(self, value, dt="f32"):
        lit = f"{value:.9e}" if dt.startswith("f") or dt == "bf16" else str(int(value))
        return self.new(f"stablehlo.constant dense<{lit}> : tensor<{dt}>")

    def splat(self, value, shape, dt="f32"):
        c = self.const(value, dt)
        return self.new(f"stablehlo.broadcast_in_dim {c}, dims = [] : (tensor<{dt}>) -> {_t(shape, dt)}")

    def bcast(self, v, src_shape, shape, dims, dt="f32"):
        return self.new(f"stablehlo.broadcast_in_dim {v}, dims = [{', '.join(map(str, dims))}] : "
                        f"({_t(src_shape, dt)}) -> {_t(shape, dt)}")

    def bin(self, op, a, b, shape, dt="f32"):
        return self.new(f"stablehlo.{op} {a}, {b} : {_t(shape, dt)}")

    def un(self, op, a, shape, dt="f32"):
        return self.new(f"stablehlo.{op} {a} : {_t(shape, dt)}")

    def convert(self, a, shape, src, dst):
        return self.new(f"stablehlo.convert {a} : ({_t(shape, src)}) -> {_t(shape, dst)}")

    def reshape(self, a, src, dst, dt):
        return self.new(f"stablehlo.reshape {a} : ({_t(src, dt)}) -> {_t(dst, dt)}")

    def transpose(self, a, src, perm, dt):
        dst = tuple(src[p] for p in perm)
        return self.new(f"stablehlo.transpose {a}, dims = [{', '.join(map(str, perm))}] : "
                        f"({_t(src, dt)}) -> {_t(dst, dt)}")

    def slice(self, a, src, starts, limits, dt):
        dst = tuple(l - s for s, l in zip(starts, limits))
        return self.new(f"stablehlo.slice {a} [{', '.join(f'{s}:{l}' for s, l in zip(starts, limits))}] : "
                        f"({_t(src, dt)}) -> {_t(dst, dt)}")

    def reduce(self, a, shape, dim, kind, init):
        dst = tuple(s for k, s in enumerate(shape) if k != dim)
        z = self.const(init)
        return self.new(f"stablehlo.reduce({a} init: {z}) applies stablehlo.{kind} across dimensions = [{dim}] : "
                        f"({_t(shape)}, tensor<f32>) -> {_t(dst)}")

    def dot(self, a, b, ashape, bshape, oshape, adt, odt, lb=(), rb=(), lc=(1,), rc=(0,)):
        bd = f"batching_dims = [{', '.join(map(str, lb))}] x [{', '.join(map(str, rb))}], " if lb else ""
        return self.new(f"stablehlo.dot_general {a}, {b}, {bd}contracting_dims = [{', '.join(map(str, lc))}] x "
                        f"[{', '.join(map(str, rc))}], precision = [DEFAULT, DEFAULT] : "
                        f"({_t(ashape, adt)}, {_t(bshape, adt)}) -> {_t(oshape, odt)}")


def _layernorm(e, x, rows, d, g, b, eps):
    """jax layer norm of x [rows, d] f32 with gamma / beta [d] (jnp.mean /
    jnp.var as reduce-sum over size, two passes), as the lowering's
    layernorm-fusion pattern expects it."""
    X, R, R1 = (rows, d), (rows,), (rows, 1)
    s = e.reduce(x, X, 1, "add", 0.0)
    s1 = e.bcast(s, R, R1, [0])
    n = e.splat(float(d), R1)
    mu = e.bin("divide", s1, n, R1)
    mub = e.bcast(mu, R1, X, [0, 1])
    xc = e.bin("subtract", x, mub, X)
    sq = e.bin("multiply", xc, xc, X)
    v = e.reduce(sq, X, 1, "add", 0.0)
    v1 = e.bcast(v, R, R1, [0])
    var = e.bin("divide", v1, n, R1)
    ve = e.bin("add", var, e.splat(float(eps), R1), R1)
    r = e.un("rsqrt", ve, R1)
    rb = e.bcast(r, R1, X, [0, 1])
    y = e.bin("multiply", xc, rb, X)
    y = e.bin("multiply", y, e.bcast(g, (d,), X, [1]), X)
    return e.bin("add", y, e.bcast(b, (d,), X, [1]), X)


def _gelu(e, x, shape):
    """jax.nn.gelu(x, approximate=True): 0.5 x (1 + tanh(c0 (x + c1 x^3)))."""
    x2 = e.bin("multiply", x, x, shape)
    x3 = e.bin("multiply", x, x2, shape)
    t = e.bin("multiply", e.splat(0.044715, shape), x3, shape)
    t = e.bin("add", x, t, shape)
    t = e.bin("multiply", e.splat(0.7978845608, shape), t, shape)
    t = e.un("tanh", t, shape)
    t = e.bin("add", e.splat(1.0, shape), t, shape)
    t = e.bin("multiply", e.splat(0.5, shape), t, shape)
    return e.bin("multiply", x, t, shape)


def _dense(e, h, w, bias, rows, k, n, gelu=False, out="bf16"):
    """jnp.dot(h, w, preferred_element_type=f32) + bias [n], GELU'd, converted."""
    y = e.dot(h, w, (rows, k), (k, n), (rows, n), "bf16", "f32")
    y = e.bin("add", y, e.bcast(bias, (n,), (rows, n), [1]), (rows, n))
    if gelu:
        y = _gelu(e, y, (rows, n))
    return e.convert(y, (rows, n), "f32", out) if out != "f32" else y


def _argmax_row(e, logits, n):
    """jnp.argmax over [1, n] f32 -> [1] i32 (variadic reduce over value and
    iota, first index on ties)."""
    I = _t((1, n), "i32")
    io = e.new(f"stablehlo.iota dim = 1 : {I}")
    ninf = e.new("stablehlo.constant dense<0xFF800000> : tensor<f32>")
    z = e.const(0, "i32")
    name = f"%v{e.n}"
    e.n += 1
    e.lines.append(f"""{e.ind}{name}:2 = "stablehlo.reduce"({logits}, {io}, {ninf}, {z}) <{{dimensions = array<i64: 1>}}> ({{
{e.ind}^bb0(%a: tensor<f32>, %ai: tensor<i32>, %b: tensor<f32>, %bi: tensor<i32>):
{e.ind}  %c0 = stablehlo.compare  GT, %a, %b,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
{e.ind}  %c1 = stablehlo.compare  NE, %a, %a,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
{e.ind}  %c2 = stablehlo.or %c0, %c1 : tensor<i1>
{e.ind}  %c3 = stablehlo.compare  EQ, %a, %b,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
{e.ind}  %c4 = stablehlo.compare  LT, %ai, %bi,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
{e.ind}  %c5 = stablehlo.and %c3, %c4 : tensor<i1>
{e.ind}  %c6 = stablehlo.or %c2, %c5 : tensor<i1>
{e.ind}  %c7 = stablehlo.select %c6, %a, %b : tensor<i1>, tensor<f32>
{e.ind}  %c8 = stablehlo.select %c6, %ai, %bi : tensor<i1>, tensor<i32>
{e.ind}  stablehlo.return %c7, %c8 : tensor<f32>, tensor<i32>
{e.ind}}}) : ({_t((1, n))}, {I}, tensor<f32>, tensor<i32>) -> ({_t((1,))}, {_t((1,), "i32")})""")
    return f"{name}#1"


def gpt_decode(c, emit_logits=False, mask_cmp="LE", trips=None):
    """Config 5 as the JAX program a user would jit (``c``: configs.GptConfig):

        def generate(ids, params):            # ids [T] i32, params as configs.gpt_param_shapes
            x = wte[ids] + wpe[:T]             # bf16 tables, f32 residual stream
            for each layer: causal self-attention (jax.nn.softmax over
                einsum scores with a tril mask), output projection, GELU MLP,
                pre-LN, writing every layer's k / v into a [H, C, hd] bf16 cache
            tok = argmax(lnf(x[T-1]) @ lm_head)
            def step(i, carry):                # lax.fori_loop over the decode steps
                x = wte[tok] + wpe[T + i]
                for each layer: q, k, v of the one row; the cache takes k, v at
                    position T + i (dynamic_update_slice); attention over the
                    cache with keys past the position masked to -inf
                tok = argmax(lnf(x) @ lm_head); out = out.at[i].set(tok)
            return tok0, out

    Inputs and outputs are those of configs.gpt_c5 (same order and types), so
    the two programs can be run on the same arrays; ``emit_logits`` adds the f32
    logits of every step [steps + 1, vocab] as a third output, as gpt_c5's does.
    ``mask_cmp`` is the comparison of the decode mask (key ``mask_cmp`` position;
    tests plant another one).  ``trips`` runs only that many decode steps (same
    inputs and outputs; for separating prefill from decode time)."""
    H, hd, D, F, T, V = c.heads, c.hd, c.d, c.mlp, c.prompt, c.vocab
    Cc = -(-c.ctx // 8) * 8
    L = c.layers
    from .configs import gpt_param_shapes
    params = gpt_param_shapes(c)
    args = [f"%ids: {_t((T,), 'i32')}"]
    pname = {}
    for k, (name, shape, dt) in enumerate(params):
        pname[name] = f"%p{k}"
        args.append(f"%p{k}: {_t(shape, dt)}")
    scale = hd ** -0.5
    e = _Emit()
    # ---- prefill
    ids2 = e.reshape("%ids", (T,), (T, 1), "i32")
    te = e.new(f'"stablehlo.gather"({pname["wte"]}, {ids2}) <{{dimension_numbers = #stablehlo.gather<offset_dims = [1], '
               f'collapsed_slice_dims = [0], start_index_map = [0], index_vector_dim = 1>, indices_are_sorted = false, '
               f'slice_sizes = array<i64: 1, {D}>}}> : ({_t((V, D), "bf16")}, {_t((T, 1), "i32")}) -> {_t((T, D), "bf16")}')
    pe = e.slice(pname["wpe"], (c.ctx, D), (0, 0), (T, D), "bf16")
    x = e.bin("add", e.convert(te, (T, D), "bf16", "f32"), e.convert(pe, (T, D), "bf16", "f32"), (T, D))
    zero = e.const(0, "i32")
    caches = []
    M_, MB = _t((T, T), "i32"), _t((T, T), "i1")
    S4, S4B = (1, H, T, T), _t((1, H, T, T), "i1")
    for l in range(L):
        p = lambda n: pname[f"h{l}.{n}"]
        h = e.convert(_layernorm(e, x, T, D, p("ln1_g"), p("ln1_b"), c.eps), (T, D), "f32", "bf16")
        qkv = _dense(e, h, p("w_qkv"), p("b_qkv"), T, D, 3 * D)
        heads = []
        for s in range(3):
            part = e.slice(qkv, (T, 3 * D), (0, s * D), (T, (s + 1) * D), "bf16")
            r = e.reshape(part, (T, D), (T, H, hd), "bf16")
            heads.append(e.transpose(r, (T, H, hd), (1, 0, 2), "bf16"))          # [H, T, hd]
        kc = e.splat(0.0, (H, Cc, hd), "bf16")
        vc = e.splat(0.0, (H, Cc, hd), "bf16")
        kc = e.new(f"stablehlo.dynamic_update_slice {kc}, {heads[1]}, {zero}, {zero}, {zero} : "
                   f"({_t((H, Cc, hd), 'bf16')}, {_t((H, T, hd), 'bf16')}, tensor<i32>, tensor<i32>, tensor<i32>) -> "
                   f"{_t((H, Cc, hd), 'bf16')}")
        vc = e.new(f"stablehlo.dynamic_update_slice {vc}, {heads[2]}, {zero}, {zero}, {zero} : "
                   f"({_t((H, Cc, hd), 'bf16')}, {_t((H, T, hd), 'bf16')}, tensor<i32>, tensor<i32>, tensor<i32>) -> "
                   f"{_t((H, Cc, hd), 'bf16')}")
        caches += [kc, vc]
        q4, k4, v4 = (e.reshape(hh, (H, T, hd), (1, H, T, hd), "bf16") for hh in heads)
        s0 = e.dot(q4, k4, (1, H, T, hd), (1, H, T, hd), S4, "bf16", "f32", lb=(0, 1), rb=(0, 1), lc=(3,), rc=(3,))
        s1 = e.bin("multiply", s0, e.splat(scale, S4), S4)
        m0 = e.new(f"stablehlo.iota dim = 0 : {M_}")
        m1 = e.new(f"stablehlo.iota dim = 1 : {M_}")
        m2 = e.new(f"stablehlo.compare  GE, {m0}, {m1},  SIGNED : ({M_}, {M_}) -> {MB}")
        m3 = e.new(f"stablehlo.broadcast_in_dim {m2}, dims = [2, 3] : ({MB}) -> {S4B}")
        ninf = e.new("stablehlo.constant dense<0xFF800000> : tensor<f32>")
        m4 = e.new(f"stablehlo.broadcast_in_dim {ninf}, dims = [] : (tensor<f32>) -> {_t(S4)}")
        s2 = e.new(f"stablehlo.select {m3}, {s1}, {m4} : {S4B}, {_t(S4)}")
        mi = e.new("stablehlo.constant dense<0xFF800000> : tensor<f32>")
        r0 = e.new(f"stablehlo.reduce({s2} init: {mi}) applies stablehlo.maximum across dimensions = [3] : "
                   f"({_t(S4)}, tensor<f32>) -> {_t((1, H, T))}")
        r1 = e.bcast(r0, (1, H, T), (1, H, T, 1), [0, 1, 2])
        r2 = e.bcast(r1, (1, H, T, 1), S4, [0, 1, 2, 3])
        ex = e.un("exponential", e.bin("subtract", s2, r2, S4), S4)
        u0 = e.reduce(ex, S4, 3, "add", 0.0)
        u1 = e.bcast(u0, (1, H, T), (1, H, T, 1), [0, 1, 2])
        u2 = e.bcast(u1, (1, H, T, 1), S4, [0, 1, 2, 3])
        pr = e.convert(e.bin("divide", ex, u2, S4), S4, "f32", "bf16")
        o0 = e.dot(pr, v4, S4, (1, H, T, hd), (1, H, T, hd), "bf16", "f32", lb=(0, 1), rb=(0, 1), lc=(3,), rc=(2,))
        o1 = e.convert(o0, (1, H, T, hd), "f32", "bf16")
        o2 = e.transpose(e.reshape(o1, (1, H, T, hd), (H, T, hd), "bf16"), (H, T, hd), (1, 0, 2), "bf16")
        att = e.reshape(o2, (T, H, hd), (T, D), "bf16")
        x = e.bin("add", x, e.bcast(p("b_o"), (D,), (T, D), [1]), (T, D))
        x = e.bin("add", x, e.dot(att, p("w_o"), (T, D), (D, D), (T, D), "bf16", "f32"), (T, D))
        h2 = e.convert(_layernorm(e, x, T, D, p("ln2_g"), p("ln2_b"), c.eps), (T, D), "f32", "bf16")
        f = _dense(e, h2, p("w_fc"), p("b_fc"), T, D, F, gelu=True)
        x = e.bin("add", x, e.bcast(p("b_proj"), (D,), (T, D), [1]), (T, D))
        x = e.bin("add", x, e.dot(f, p("w_proj"), (T, F), (F, D), (T, D), "bf16", "f32"), (T, D))
    last = e.slice(x, (T, D), (T - 1, 0), (T, D), "f32")

    hf0 = e.convert(_layernorm(e, last, 1, D, pname["lnf_g"], pname["lnf_b"], c.eps), (1, D), "f32", "bf16")
    lg0 = e.dot(hf0, pname["lm_head"], (1, D), (D, V), (1, V), "bf16", "f32")
    tok0 = _argmax_row(e, lg0, V)
    # ---- decode loop
    out0 = e.splat(0, (c.steps,), "i32")
    i0 = e.const(0, "i32")
    KV = _t((H, Cc, hd), "bf16")
    LG = _t((c.steps + 1, V))
    ctypes_ = ["tensor<i32>", _t((1,), "i32"), _t((c.steps,), "i32")] + [KV] * (2 * L)
    cvals = [i0, tok0, out0] + caches
    bargs = ["%i", "%tok", "%out"] + [f"%c{k}" for k in range(2 * L)]
    if emit_logits:
        lz = e.splat(0.0, (c.steps + 1, V))
        lg_all = e.new(f"stablehlo.dynamic_update_slice {lz}, {lg0}, {i0}, {i0} : ({LG}, {_t((1, V))}, "
                       f"tensor<i32>, tensor<i32>) -> {LG}")
        ctypes_.append(LG)
        cvals.append(lg_all)
        bargs.append("%lg")
    b = _Emit(indent="      ")
    one = b.const(1, "i32")
    pos = b.new(f"stablehlo.add %i, {b.const(T, 'i32')} : tensor<i32>")
    bz = b.const(0, "i32")
    t2 = b.reshape("%tok", (1,), (1, 1), "i32")
    te1 = b.new(f'"stablehlo.gather"({pname["wte"]}, {t2}) <{{dimension_numbers = #stablehlo.gather<offset_dims = [1], '
                f'collapsed_slice_dims = [0], start_index_map = [0], index_vector_dim = 1>, indices_are_sorted = false, '
                f'slice_sizes = array<i64: 1, {D}>}}> : ({_t((V, D), "bf16")}, {_t((1, 1), "i32")}) -> {_t((1, D), "bf16")}')
    pe1 = b.new(f"stablehlo.dynamic_slice {pname['wpe']}, {pos}, {bz}, sizes = [1, {D}] : "
                f"({_t((c.ctx, D), 'bf16')}, tensor<i32>, tensor<i32>) -> {_t((1, D), 'bf16')}")
    xs = b.bin("add", b.convert(te1, (1, D), "bf16", "f32"), b.convert(pe1, (1, D), "bf16", "f32"), (1, D))
    new_caches = []
    S3 = (H, 1, Cc)
    for l in range(L):
        p = lambda n: pname[f"h{l}.{n}"]
        h = b.convert(_layernorm(b, xs, 1, D, p("ln1_g"), p("ln1_b"), c.eps), (1, D), "f32", "bf16")
        qkv = _dense(b, h, p("w_qkv"), p("b_qkv"), 1, D, 3 * D)
        q, k, v = (b.reshape(b.slice(qkv, (1, 3 * D), (0, s * D), (1, (s + 1) * D), "bf16"), (1, D), (H, 1, hd), "bf16")
                   for s in range(3))
        kc = b.new(f"stablehlo.dynamic_update_slice %c{2 * l}, {k}, {bz}, {pos}, {bz} : ({KV}, {_t((H, 1, hd), 'bf16')}, "
                   f"tensor<i32>, tensor<i32>, tensor<i32>) -> {KV}")
        vc = b.new(f"stablehlo.dynamic_update_slice %c{2 * l + 1}, {v}, {bz}, {pos}, {bz} : ({KV}, {_t((H, 1, hd), 'bf16')}, "
                   f"tensor<i32>, tensor<i32>, tensor<i32>) -> {KV}")
        new_caches += [kc, vc]
        sc = b.dot(q, kc, (H, 1, hd), (H, Cc, hd), S3, "bf16", "f32", lb=(0,), rb=(0,), lc=(2,), rc=(2,))
        sc = b.bin("multiply", sc, b.splat(scale, S3), S3)
        io = b.new(f"stablehlo.iota dim = 2 : {_t(S3, 'i32')}")
        pb = b.new(f"stablehlo.broadcast_in_dim {pos}, dims = [] : (tensor<i32>) -> {_t(S3, 'i32')}")
        vis = b.new(f"stablehlo.compare  {mask_cmp}, {io}, {pb},  SIGNED : ({_t(S3, 'i32')}, {_t(S3, 'i32')}) -> "
                    f"{_t(S3, 'i1')}")
        ni = b.new("stablehlo.constant dense<0xFF800000> : tensor<f32>")
        nib = b.new(f"stablehlo.broadcast_in_dim {ni}, dims = [] : (tensor<f32>) -> {_t(S3)}")
        sm = b.new(f"stablehlo.select {vis}, {sc}, {nib} : {_t(S3, 'i1')}, {_t(S3)}")
        mi = b.new("stablehlo.constant dense<0xFF800000> : tensor<f32>")
        mx = b.new(f"stablehlo.reduce({sm} init: {mi}) applies stablehlo.maximum across dimensions = [2] : "
                   f"({_t(S3)}, tensor<f32>) -> {_t((H, 1))}")
        mxb = b.bcast(mx, (H, 1), S3, [0, 1])
        ex = b.un("exponential", b.bin("subtract", sm, mxb, S3), S3)
        sm1 = b.reduce(ex, S3, 2, "add", 0.0)
        pr = b.convert(b.bin("divide", ex, b.bcast(sm1, (H, 1), S3, [0, 1]), S3), S3, "f32", "bf16")
        o = b.dot(pr, vc, S3, (H, Cc, hd), (H, 1, hd), "bf16", "f32", lb=(0,), rb=(0,), lc=(2,), rc=(1,))
        att = b.reshape(b.convert(o, (H, 1, hd), "f32", "bf16"), (H, 1, hd), (1, D), "bf16")
        xs = b.bin("add", xs, b.bcast(p("b_o"), (D,), (1, D), [1]), (1, D))
        xs = b.bin("add", xs, b.dot(att, p("w_o"), (1, D), (D, D), (1, D), "bf16", "f32"), (1, D))
        h2 = b.convert(_layernorm(b, xs, 1, D, p("ln2_g"), p("ln2_b"), c.eps), (1, D), "f32", "bf16")
        f = _dense(b, h2, p("w_fc"), p("b_fc"), 1, D, F, gelu=True)
        xs = b.bin("add", xs, b.bcast(p("b_proj"), (D,), (1, D), [1]), (1, D))
        xs = b.bin("add", xs, b.dot(f, p("w_proj"), (1, F), (F, D), (1, D), "bf16", "f32"), (1, D))
    hf = b.convert(_layernorm(b, xs, 1, D, pname["lnf_g"], pname["lnf_b"], c.eps), (1, D), "f32", "bf16")
    lg = b.dot(hf, pname["lm_head"], (1, D), (D, V), (1, V), "bf16", "f32")
    tok = _argmax_row(b, lg, V)
    out = b.new(f"stablehlo.dynamic_update_slice %out, {tok}, %i : ({_t((c.steps,), 'i32')}, {_t((1,), 'i32')}, "
                f"tensor<i32>) -> {_t((c.steps,), 'i32')}")
    i1 = b.new(f"stablehlo.add %i, {one} : tensor<i32>")
    rets = [i1, tok, out] + new_caches
    if emit_logits:
        rets.append(b.new(f"stablehlo.dynamic_update_slice %lg, {lg}, {i1}, {bz} : ({LG}, {_t((1, V))}, "
                          f"tensor<i32>, tensor<i32>) -> {LG}"))
    nres = len(cvals)
    blockargs = ", ".join(f"{n}: {ty}" for n, ty in zip(bargs, ctypes_))
    types = ", ".join(ctypes_)
    loop = f"""    %w:{nres} = "stablehlo.while"({', '.join(cvals)}) ({{
    ^bb0({blockargs}):
      %lim = stablehlo.constant dense<{c.steps if trips is None else trips}> : tensor<i32>
      %lt = stablehlo.compare  LT, %i, %lim,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
      stablehlo.return %lt : tensor<i1>
    }}, {{
    ^bb0({blockargs}):
{chr(10).join(b.lines)}
      stablehlo.return {', '.join(rets)} : {types}
    }}) : ({types}) -> ({types})"""
    body = "\n".join(e.lines) + "\n" + loop
    R1, RS = _t((1,), "i32"), _t((c.steps,), "i32")
    res, rty = [tok0, "%w#2"], [R1, RS]
    if emit_logits:
        res.append(f"%w#{nres - 1}")
        rty.append(LG)
    return f"""
module @jit_generate {{
  func.func public @main({', '.join(args)}) -> ({', '.join(rty)}) {{
{body}
    return {', '.join(res)} : {', '.join(rty)}
  }}
}}
"""


# ---- the reference's decode benchmark step ---------------------------------------------------

DECODE_STEP_CONFIGS = {              # (d_model, heads, d_ff, layers, context): tools/bench_decode.py:21-31
    "small": (256, 4, 1024, 4, 128),
    "base": (512, 8, 2048, 6, 256),
    "large": (1024, 16, 4096, 6, 512),
}
DECODE_STEP_KEYS = ("ln1_b", "ln1_g", "ln2_b", "ln2_g", "w1", "w2", "wk", "wo", "wq", "wv")


def decode_step_params(cfg):
    """[(name, shape)] of the step's f32 inputs in jit argument order: x, kc,
    vc, then each layer's parameter dict flattened by sorted key (JAX's pytree
    order for a dict)."""
    D, H, F, L, C = cfg
    hd = D // H
    shapes = {"ln1_b": (D,), "ln1_g": (D,), "ln2_b": (D,), "ln2_g": (D,), "w1": (D, F), "w2": (F, D),
              "wk": (D, D), "wo": (D, D), "wq": (D, D), "wv": (D, D)}
    out = [("x", (1, D)), ("kc", (L, H, C, hd)), ("vc", (L, H, C, hd))]
    for l in range(L):
        out += [(f"{l}.{k}", shapes[k]) for k in DECODE_STEP_KEYS]
    return out


def decode_step(cfg):
    """One token of tools/bench_decode.py:35-65 (the reference's decode
    benchmark), f32 throughout, ``cfg`` = (d_model, heads, d_ff, layers, C):

        def step(x, kc, vc, params):          # x (1, D); kc, vc (L, H, C, hd)
            for li, p in enumerate(params):
                h = ln(x, p["ln1_g"], p["ln1_b"])       # mean / var by .mean(), (v + eps) ** -0.5
                q, k, v = ((h @ p[w]).reshape(H, 1, hd) for w in ("wq", "wk", "wv"))
                kk = jnp.concatenate([kc[li], k], axis=1)  # (H, C + 1, hd)
                vv = jnp.concatenate([vc[li], v], axis=1)
                a = softmax((q @ jnp.swapaxes(kk, -1, -2)) * hd ** -0.5)
                x = x + (a @ vv).reshape(1, D) @ p["wo"]
                h = ln(x, p["ln2_g"], p["ln2_b"])
                x = x + gelu(h @ p["w1"]) @ p["w2"]   # 0.5 x (1 + tanh(c (x + 0.044715 x ** 3)))
            return x"""
    D, H, F, L, C = cfg
    hd = D // H
    params = decode_step_params(cfg)
    pname = {n: f"%a{k}" for k, (n, _) in enumerate(params)}
    args = [f"%a{k}: {_t(s)}" for k, (_, s) in enumerate(params)]
    e = _Emit()
    X, R1 = (1, D), (1, 1)

    def mean_keep(v, shape):
        s = e.reduce(v, shape, 1, "add", 0.0)
        s = e.bin("divide", s, e.splat(float(shape[1]), (1,)), (1,))
        return e.reshape(s, (1,), R1, "f32")

    def ln(x, g, b):
        m = mean_keep(x, X)
        xc = e.bin("subtract", x, e.bcast(m, R1, X, [0, 1]), X)
        v = mean_keep(e.bin("multiply", xc, xc, X), X)
        ve = e.bin("add", v, e.splat(1e-5, R1), R1)
        r = e.bin("power", ve, e.splat(-0.5, R1), R1)
        y = e.bin("multiply", xc, e.bcast(r, R1, X, [0, 1]), X)
        y = e.bin("multiply", y, e.bcast(g, (D,), X, [1]), X)
        return e.bin("add", y, e.bcast(b, (D,), X, [1]), X)

    def mm(a, w, k, n):
        return e.dot(a, w, (1, k), (k, n), (1, n), "f32", "f32")

    x = pname["x"]
    S3, KK = (H, 1, C + 1), (H, C + 1, hd)
    for l in range(L):
        p = lambda n: pname[f"{l}.{n}"]
        h = ln(x, p("ln1_g"), p("ln1_b"))
        q, k, v = (e.reshape(mm(h, p(w), D, D), X, (H, 1, hd), "f32") for w in ("wq", "wk", "wv"))
        parts = []
        for cache, new in (("kc", k), ("vc", v)):
            sl = e.slice(pname[cache], (L, H, C, hd), (l, 0, 0, 0), (l + 1, H, C, hd), "f32")
            sl = e.reshape(sl, (1, H, C, hd), (H, C, hd), "f32")
            parts.append(e.new(f"stablehlo.concatenate {sl}, {new}, dim = 1 : ({_t((H, C, hd))}, "
                               f"{_t((H, 1, hd))}) -> {_t(KK)}"))
        kk, vv = parts
        kt = e.transpose(kk, KK, (0, 2, 1), "f32")
        s = e.dot(q, kt, (H, 1, hd), (H, hd, C + 1), S3, "f32", "f32", lb=(0,), rb=(0,), lc=(2,), rc=(1,))
        s = e.bin("multiply", s, e.splat(hd ** -0.5, S3), S3)
        mi = e.new("stablehlo.constant dense<0xFF800000> : tensor<f32>")
        mx = e.new(f"stablehlo.reduce({s} init: {mi}) applies stablehlo.maximum across dimensions = [2] : "
                   f"({_t(S3)}, tensor<f32>) -> {_t((H, 1))}")
        mx = e.reshape(mx, (H, 1), (H, 1, 1), "f32")
        ex = e.un("exponential", e.bin("subtract", s, e.bcast(mx, (H, 1, 1), S3, [0, 1, 2]), S3), S3)
        sm = e.reshape(e.reduce(ex, S3, 2, "add", 0.0), (H, 1), (H, 1, 1), "f32")
        a = e.bin("divide", ex, e.bcast(sm, (H, 1, 1), S3, [0, 1, 2]), S3)
        o = e.dot(a, vv, S3, KK, (H, 1, hd), "f32", "f32", lb=(0,), rb=(0,), lc=(2,), rc=(1,))
        o = e.reshape(o, (H, 1, hd), X, "f32")
        x = e.bin("add", x, mm(o, p("wo"), D, D), X)
        h = ln(x, p("ln2_g"), p("ln2_b"))
        f = mm(h, p("w1"), D, F)
        F2 = (1, F)
        f3 = e.bin("multiply", e.bin("multiply", f, f, F2), f, F2)
        t = e.bin("add", f, e.bin("multiply", e.splat(0.044715, F2), f3, F2), F2)
        t = e.un("tanh", e.bin("multiply", e.splat(0.7978845608, F2), t, F2), F2)
        t = e.bin("add", e.splat(1.0, F2), t, F2)
        g = e.bin("multiply", e.bin("multiply", e.splat(0.5, F2), f, F2), t, F2)
        x = e.bin("add", x, mm(g, p("w2"), F, D), X)
    body = "\n".join(e.lines)
    return f"""
module @jit__lambda_ {{
  func.func public @main({', '.join(args)}) -> ({_t(X)}) {{
{body}
    return {x} : {_t(X)}
  }}
}}
"""


def decode_step_inputs(cfg, seed=0):
    """Inputs of decode_step in its argument order, drawn as
    tools/bench_decode.py:68-80 draws them (weights, caches ~ N(0, 0.02), x ~
    N(0, 1), layernorm gains 1 and shifts 0; numpy's generator, not the same
    stream)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    out = []
    for name, shape in decode_step_params(cfg):
        key = name.split(".")[-1]
        if key in ("ln1_g", "ln2_g"):
            out.append(np.ones(shape, np.float32))
        elif key in ("ln1_b", "ln2_b"):
            out.append(np.zeros(shape, np.float32))
        else:
            out.append((rng.standard_normal(shape) * (1.0 if name == "x" else 0.02)).astype(np.float32))
    return out


def decode_step_bytes(cfg) -> int:
    """Bytes one step must read (tools/bench_decode.py:83-89): the f32 weights
    once and the two caches."""
    D, H, F, L, C = cfg
    return L * (4 * D * D + 2 * D * F) * 4 + L * 2 * H * C * (D // H) * 4
