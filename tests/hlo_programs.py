"""StableHLO programs, as MLIR text in the form JAX prints them (``jax.jit(f)
.lower(...).as_text()``), for the lowering tests.  Each builder returns the text
for the given sizes; the comment above it is the JAX function it stands for.

jax is not installed in this image, so these texts are written out by hand
following JAX's lowering rules (jnp.mean = reduce-sum / size, integer_pow by
repeated squaring, jax.nn.softmax = exp(x - max) / sum, jnp.argmax = a
variadic reduce over (value, iota)); which exact StableHLO a given JAX version
emits is not pinned here."""


import numpy as np

from pjrt_amd.stablehlo_configs import _t, attention, ln_gelu, matmul, mlp  # noqa: F401


def argmax_rows(rows=4, n=1000):
    """def f(x): return jnp.max(x, -1), jnp.argmax(x, -1).astype(jnp.int32)"""
    X, R, RI, I = _t((rows, n)), _t((rows,)), _t((rows,), "i32"), _t((rows, n), "i32")
    return f"""
module @jit_f {{
  func.func public @main(%arg0: {X}) -> ({R}, {RI}) {{
    %0 = stablehlo.iota dim = 1 : {I}
    %cst = stablehlo.constant dense<0xFF800000> : tensor<f32>
    %c = stablehlo.constant dense<0> : tensor<i32>
    %1:2 = "stablehlo.reduce"(%arg0, %0, %cst, %c) <{{dimensions = array<i64: 1>}}> ({{
    ^bb0(%a: tensor<f32>, %ai: tensor<i32>, %b: tensor<f32>, %bi: tensor<i32>):
      %2 = stablehlo.compare  GT, %a, %b,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
      %3 = stablehlo.compare  NE, %a, %a,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
      %4 = stablehlo.or %2, %3 : tensor<i1>
      %5 = stablehlo.compare  EQ, %a, %b,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
      %6 = stablehlo.compare  LT, %ai, %bi,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
      %7 = stablehlo.and %5, %6 : tensor<i1>
      %8 = stablehlo.or %4, %7 : tensor<i1>
      %9 = stablehlo.select %8, %a, %b : tensor<i1>, tensor<f32>
      %10 = stablehlo.select %8, %ai, %bi : tensor<i1>, tensor<i32>
      stablehlo.return %9, %10 : tensor<f32>, tensor<i32>
    }}) : ({X}, {I}, tensor<f32>, tensor<i32>) -> ({R}, {RI})
    return %1#0, %1#1 : {R}, {RI}
  }}
}}
"""


def fori_add(trips=5, n=1):
    """def f(x): return lax.fori_loop(0, trips, lambda i, a: a + 3.0, x)
    (reference tests/_while_e2e_body.py: fori_loop(0, 5, +3) from 2 -> 17)"""
    X = _t((n,)) if n > 1 else "tensor<f32>"
    return f"""
module @jit_f {{
  func.func public @main(%arg0: {X}) -> {X} {{
    %c = stablehlo.constant dense<0> : tensor<i32>
    %0:2 = "stablehlo.while"(%c, %arg0) ({{
    ^bb0(%i: tensor<i32>, %a: {X}):
      %lim = stablehlo.constant dense<{trips}> : tensor<i32>
      %1 = stablehlo.compare  LT, %i, %lim,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
      stablehlo.return %1 : tensor<i1>
    }}, {{
    ^bb0(%i: tensor<i32>, %a: {X}):
      %one = stablehlo.constant dense<1> : tensor<i32>
      %2 = stablehlo.add %i, %one : tensor<i32>
      %three = stablehlo.constant dense<3.000000e+00> : tensor<f32>
      %3 = stablehlo.broadcast_in_dim %three, dims = [] : (tensor<f32>) -> {X}
      %4 = stablehlo.add %a, %3 : {X}
      stablehlo.return %2, %4 : tensor<i32>, {X}
    }}) : (tensor<i32>, {X}) -> (tensor<i32>, {X})
    return %0#1 : {X}
  }}
}}
"""


def while_double():
    """def f(v): return lax.while_loop(lambda c: c[1] < 1000.0, lambda c: (c[0] + 1, c[1] * 2), (0, v))
    (a data-dependent loop: 1.0 -> (10, 1024.0), the reference's while-doubling answer)"""
    return """
module @jit_f {
  func.func public @main(%arg0: tensor<f32>) -> (tensor<i32>, tensor<f32>) {
    %c = stablehlo.constant dense<0> : tensor<i32>
    %0:2 = "stablehlo.while"(%c, %arg0) ({
    ^bb0(%i: tensor<i32>, %v: tensor<f32>):
      %lim = stablehlo.constant dense<1.000000e+03> : tensor<f32>
      %1 = stablehlo.compare  LT, %v, %lim,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
      stablehlo.return %1 : tensor<i1>
    }, {
    ^bb0(%i: tensor<i32>, %v: tensor<f32>):
      %one = stablehlo.constant dense<1> : tensor<i32>
      %2 = stablehlo.add %i, %one : tensor<i32>
      %two = stablehlo.constant dense<2.000000e+00> : tensor<f32>
      %3 = stablehlo.multiply %v, %two : tensor<f32>
      stablehlo.return %2, %3 : tensor<i32>, tensor<f32>
    }) : (tensor<i32>, tensor<f32>) -> (tensor<i32>, tensor<f32>)
    return %0#0, %0#1 : tensor<i32>, tensor<f32>
  }
}
"""


def scan_stack(trips=6, n=4):
    """def f(x):   # lax.scan stacking: ys[i] = x * (i + 1)
         def body(c, _):
             i, ys = c
             ys = lax.dynamic_update_slice(ys, (x * (i + 1).astype(jnp.float32))[None], (i, 0))
             return (i + 1, ys), None
         return lax.fori_loop(0, trips, ..., (0, zeros((trips, n))))[1]"""
    X, Y, Y1 = _t((n,)), _t((trips, n)), _t((1, n))
    return f"""
module @jit_f {{
  func.func public @main(%arg0: {X}) -> {Y} {{
    %c = stablehlo.constant dense<0> : tensor<i32>
    %z = stablehlo.constant dense<0.000000e+00> : {Y}
    %0:3 = "stablehlo.while"(%c, %z, %arg0) ({{
    ^bb0(%i: tensor<i32>, %ys: {Y}, %x: {X}):
      %lim = stablehlo.constant dense<{trips}> : tensor<i32>
      %1 = stablehlo.compare  LT, %i, %lim,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
      stablehlo.return %1 : tensor<i1>
    }}, {{
    ^bb0(%i: tensor<i32>, %ys: {Y}, %x: {X}):
      %one = stablehlo.constant dense<1> : tensor<i32>
      %2 = stablehlo.add %i, %one : tensor<i32>
      %3 = stablehlo.convert %2 : (tensor<i32>) -> tensor<f32>
      %4 = stablehlo.broadcast_in_dim %3, dims = [] : (tensor<f32>) -> {X}
      %5 = stablehlo.multiply %x, %4 : {X}
      %6 = stablehlo.reshape %5 : ({X}) -> {Y1}
      %zc = stablehlo.constant dense<0> : tensor<i32>
      %7 = stablehlo.dynamic_update_slice %ys, %6, %i, %zc : ({Y}, {Y1}, tensor<i32>, tensor<i32>) -> {Y}
      stablehlo.return %2, %7, %x : tensor<i32>, {Y}, {X}
    }}) : (tensor<i32>, {Y}, {X}) -> (tensor<i32>, {Y}, {X})
    return %0#1 : {Y}
  }}
}}
"""


def generic_chain(n=64):
    """The generic op form (what an MLIR printer emits with
    print_generic_op_form=True): y = exp(x) * 2 - x, then a transpose."""
    X = _t((n // 8, 8))
    XT = _t((8, n // 8))
    return f"""
"builtin.module"() <{{sym_name = "jit_f"}}> ({{
  "func.func"() <{{function_type = ({X}) -> {XT}, sym_name = "main", sym_visibility = "public"}}> ({{
  ^bb0(%arg0: {X}):
    %0 = "stablehlo.exponential"(%arg0) : ({X}) -> {X}
    %1 = "stablehlo.constant"() <{{value = dense<2.000000e+00> : tensor<f32>}}> : () -> tensor<f32>
    %2 = "stablehlo.broadcast_in_dim"(%1) <{{broadcast_dimensions = array<i64>}}> : (tensor<f32>) -> {X}
    %3 = "stablehlo.multiply"(%0, %2) : ({X}, {X}) -> {X}
    %4 = "stablehlo.subtract"(%3, %arg0) : ({X}, {X}) -> {X}
    %5 = "stablehlo.transpose"(%4) <{{permutation = array<i64: 1, 0>}}> : ({X}) -> {XT}
    "func.return"(%5) : ({XT}) -> ()
  }}) : () -> ()
}}) {{mhlo.num_partitions = 1 : i32}} : () -> ()
"""


def donated_chain(n=64, alias_to=0, twice=True):
    """def f(x, w): return (x @ w) @ w  with jax.jit(f, donate_argnums=0): the
    donated x carries tf.aliasing_output.  twice=False: return x + w (read and
    written in the same phase)."""
    X = _t((n, n))
    body = f"""
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : ({X}, {X}) -> {X}
    %1 = stablehlo.dot_general %0, %arg1, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : ({X}, {X}) -> {X}
    return %1 : {X}""" if twice else f"""
    %1 = stablehlo.add %arg0, %arg1 : {X}
    return %1 : {X}"""
    return f"""
module @jit_f {{
  func.func public @main(%arg0: {X} {{tf.aliasing_output = {alias_to} : i32}}, %arg1: {X}) -> ({X} {{jax.result_info = ""}}) {{{body}
  }}
}}
"""


def fori_shift(trips=5, swap=False):
    """def f(x):   # a carry passed on while another is updated
         return lax.fori_loop(0, trips, lambda i, c: (c[0] + 1.0, c[0]), (x, -x))
    -> (x + trips, x + trips - 1): the second carry must see the first one's
    value from before the update.  With ``swap`` the body is
    ``lambda i, c: (c[1], c[0])``."""
    ret = "%b, %a" if swap else "%3, %a"
    return f"""
module @jit_f {{
  func.func public @main(%arg0: tensor<f32>) -> (tensor<f32>, tensor<f32>) {{
    %c = stablehlo.constant dense<0> : tensor<i32>
    %n = stablehlo.negate %arg0 : tensor<f32>
    %0:3 = "stablehlo.while"(%c, %arg0, %n) ({{
    ^bb0(%i: tensor<i32>, %a: tensor<f32>, %b: tensor<f32>):
      %lim = stablehlo.constant dense<{trips}> : tensor<i32>
      %1 = stablehlo.compare  LT, %i, %lim,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
      stablehlo.return %1 : tensor<i1>
    }}, {{
    ^bb0(%i: tensor<i32>, %a: tensor<f32>, %b: tensor<f32>):
      %one = stablehlo.constant dense<1> : tensor<i32>
      %2 = stablehlo.add %i, %one : tensor<i32>
      %f1 = stablehlo.constant dense<1.000000e+00> : tensor<f32>
      %3 = stablehlo.add %a, %f1 : tensor<f32>
      stablehlo.return %2, {ret} : tensor<i32>, tensor<f32>, tensor<f32>
    }}) : (tensor<i32>, tensor<f32>, tensor<f32>) -> (tensor<i32>, tensor<f32>, tensor<f32>)
    return %0#1, %0#2 : tensor<f32>, tensor<f32>
  }}
}}
"""


def decode_step_reference(cfg, arrays):
    """tools/bench_decode.py:35-65 restated in float64 numpy: one decode token
    through the layers, keys and values appended to the caches."""
    from pjrt_amd import stablehlo_configs as SC
    D, H, F, L, C = cfg
    hd = D // H
    P = {n: a.astype(np.float64) for (n, _), a in zip(SC.decode_step_params(cfg), arrays)}
    x, kc, vc = P["x"], P["kc"], P["vc"]

    def ln(x, g, b):
        m = x.mean(-1, keepdims=True)
        v = ((x - m) ** 2).mean(-1, keepdims=True)
        return (x - m) / np.sqrt(v + 1e-5) * g + b

    def gelu(x):
        return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))

    for l in range(L):
        p = lambda n: P[f"{l}.{n}"]
        h = ln(x, p("ln1_g"), p("ln1_b"))
        q, k, v = ((h @ p(w)).reshape(H, 1, hd) for w in ("wq", "wk", "wv"))
        kk = np.concatenate([kc[l], k], 1)
        vv = np.concatenate([vc[l], v], 1)
        s = q @ kk.transpose(0, 2, 1) * hd ** -0.5
        a = np.exp(s - s.max(-1, keepdims=True))
        a /= a.sum(-1, keepdims=True)
        x = x + (a @ vv).reshape(1, D) @ p("wo")
        x = x + gelu(ln(x, p("ln2_g"), p("ln2_b")) @ p("w1")) @ p("w2")
    return x
