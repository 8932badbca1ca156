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
