"""The compiled-model runtime on the GPU (lk.compile / lk.load / compile_ir over include/lokinfer_rt.h): traced
models against the same ops run eagerly, bit for bit (same kernels, same order); .lkm save / load round trips;
symbolic shapes bound per call (one captured hipGraph per binding); data-dependent shapes (dim.read); persistent
state written in place; errors from kernels, shapes and the device error record."""
import numpy as np
import pytest
import torch

from lokinfer_amd._lib import LokinferError

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(11)


def G(lk, a, dt=np.float32):
    return lk.from_numpy(np.ascontiguousarray(a, dt), device="gpu", copy=True)


def mlp_params(lk):
    from oracle import mnist

    x, (w1, b1, w2, b2) = mnist.mlp_inputs(1)
    return x, [G(lk, p) for p in (w1, b1, w2, b2)], (w1, b1, w2, b2)


def test_mnist_mlp_compiled_equals_eager_and_oracle(gpu, tmp_path):
    lk = gpu
    from oracle import mnist

    x, (W1, B1, W2, B2), params = mlp_params(lk)

    def mlp(xx):
        return lk.ops.gemm_bias_f32_gpu(lk.ops.gemm_bias_relu_f32_gpu(xx, W1, B1), W2, B2)

    X = G(lk, x)
    eager = mlp(X).numpy()
    m = lk.compile(mlp, inputs=[X])
    assert 'kernel "gemm_bias_relu_f32_gpu"' in m.source_ir and m.num_external_constants == 4
    for _ in range(3):  # first call eager in the call block, later calls replay the captured graph
        assert np.array_equal(m(X).numpy(), eager)
    assert m.stats()["graphs"] == 1
    ref = mnist.mlp_forward(x, params)
    assert np.abs(eager - ref).max() <= 1e-4 * np.abs(ref).max()
    path = tmp_path / "mlp.lkm"
    m.save(path)
    m2 = lk.load(path)
    assert np.array_equal(m2(X).numpy(), eager)
    assert 'const.internal @"ext0"' in m2.ir_text()


def test_traced_stream_structure_replayed(gpu):
    """A function that runs branches on side streams (GpuContext.branch / join / mark / wait_mark) leaves its stream
    structure in the IR (lane, seq, after); the executable captures each lane on its own stream with those waits
    plus the data dependencies. The replays equal the eager run bit for bit, with other work between them."""
    from lokinfer_amd.runtime import GpuContext

    lk = gpu
    ctx = GpuContext.shared()
    side = [torch.cuda.Stream() for _ in range(2)]
    D = 256
    w1, w2, w3 = (G(lk, rng.standard_normal((D, D)) / 16) for _ in range(3))
    b = G(lk, 0.1 * rng.standard_normal(D))

    def f(x):
        h = lk.ops.gemm_bias_f32_gpu(x, w1, b)
        with ctx.branch(side[0], 1):  # a branch of two dependent kernels, marked half way
            u = lk.ops.gemm_f32_gpu_mps(h, w2)
            m = ctx.mark(side[0])
            u = lk.ops.leaky_lc_f32_gpu(u, 0.2)
        with ctx.branch(side[1], 2):  # waits for the branch's first kernel only
            ctx.wait_mark(side[1], m)
            v = lk.ops.gemm_f32_gpu_mps(h, w3)
        y = lk.ops.gemm_f32_gpu_mps(h, w1)
        ctx.join(side[0])
        ctx.join(side[1])
        return lk.ops.add3_scale_f32_gpu(y, u, v, 0.5)

    X = G(lk, rng.standard_normal((300, D)))
    eager = f(X).numpy()
    cm = lk.compile(f, inputs=[X], lanes=4)
    ir = cm.source_ir
    assert 'lane = "1"' in ir and 'lane = "2"' in ir and 'after = "' in ir
    for _ in range(4):
        assert np.array_equal(cm(X).numpy(), eager)
        lk.ops.gemm_f32_gpu_mps(X, w2).numpy()  # eager work between the replays
    assert cm.stats()["graphs"] == 1 and cm.stats()["lanes"] == 3


def test_symbolic_rows_one_graph_per_binding(gpu):
    lk = gpu
    D = 256
    gamma, beta = G(lk, 1 + 0.1 * rng.standard_normal(D)), G(lk, 0.1 * rng.standard_normal(D))
    w = G(lk, rng.standard_normal((D, 3 * D)) / 16)

    def f(x):
        h = lk.ops.layernorm_f32_gpu(x, gamma, beta)
        y = lk.ops.gemm_f32_gpu_mps(h, w)
        return lk.ops.view(y, [x.shape[0], D], 0), y  # a view of the first D columns' worth of elements

    T = lk.Sym("T")
    m = lk.compile(f, input_types=[lk.TensorType(lk.f32, [T, D])])
    assert "exec(%in0_1: buffer<f32[T, 256]>)" in m.ir_text()
    for t in (5, 37, 5, 128):
        X = G(lk, rng.standard_normal((t, D)))
        v, y = m(X)
        ye = lk.ops.gemm_f32_gpu_mps(lk.ops.layernorm_f32_gpu(X, gamma, beta), w).numpy()
        assert y.shape == (t, 3 * D) and np.array_equal(y.numpy(), ye)
        assert np.array_equal(v.numpy(), ye.reshape(-1)[: t * D].reshape(t, D))
    assert m.stats()["graphs"] == 3


def test_data_dependent_shape_dim_read(gpu):
    """F = argmax of a row (read on the host with dim.read), then a GEMM over the first F rows: an eager call
    whose shapes are bound mid-call."""
    lk = gpu
    w = G(lk, rng.standard_normal((64, 32)))

    def f(scores, rows):
        idx = lk.ops.argmax_f32_gpu(scores)  # i64[1]
        F = lk.dim_read(lk.ops.to_cpu(idx), 0, "F")
        head = lk.ops.view(rows, [F, 64], 0)
        return lk.ops.gemm_f32_gpu_mps(head, w)

    m = lk.compile(f, input_types=[lk.TensorType(lk.f32, [1, 100]), lk.TensorType(lk.f32, [100, 64])])
    assert "dim.read" in m.ir_text()
    for k in (7, 63, 1):
        s = np.zeros((1, 100), np.float32)
        s[0, k] = 1
        rows = rng.standard_normal((100, 64)).astype(np.float32)
        got = m(G(lk, s), G(lk, rows)).numpy()
        assert got.shape == (k, 32)
        assert np.array_equal(got, lk.ops.gemm_f32_gpu_mps(G(lk, rows[:k]), w).numpy())
    assert m.stats()["graphs"] == 0


def test_dim_read_index_checked_against_a_symbolic_extent(gpu):
    """dim.read's index is checked at run time when its operand's extent is symbolic (the verifier can only check
    static ones): element 5 of an i64[N] input reads fine at N = 8 and is an error at N = 3."""
    lk = gpu
    ir = """model {
  init {
    return
  }
  exec(%x: tensor<i64[N]>, %a: tensor<f32[N]>) {
    dim.read %x[5] -> F
    %b = kernel "add_f32_gpu"(%a, %a) : tensor<f32[N]>
    return %b
  }
}
"""
    m = lk.compile_ir(ir)
    got = m(G(lk, np.arange(8), np.int64), G(lk, np.ones(8))).numpy()
    assert np.array_equal(got, np.full(8, 2.0, np.float32))
    with pytest.raises(LokinferError, match="outside its operand"):
        m(G(lk, np.arange(3), np.int64), G(lk, np.ones(3)))


def test_persistent_kv_cache_written_in_place(gpu):
    """A decode step over persistent caches (model state, hoisted into init, zeroed at create) equals the same
    ops over caller caches, step after step."""
    lk = gpu
    from lokinfer_amd.graph import TensorType

    heads, cap, D = 4, 64, 256
    bias = G(lk, 0.1 * rng.standard_normal(3 * D))

    def step(qkv, pos):
        g = lk.graph.current_graph()
        kc = g.persistent(TensorType(lk.f32, [cap, D]))
        vc = g.persistent(TensorType(lk.f32, [cap, D]))
        return lk.ops.attention_decode_f32_gpu(qkv, kc, vc, pos, bias, heads)

    m = lk.compile(step, input_types=[TensorType(lk.f32, [1, 3 * D]), TensorType(lk.i64, [1])])
    assert "persistent = true" in m.ir_text()
    KC, VC = G(lk, np.zeros((cap, D))), G(lk, np.zeros((cap, D)))
    for p in range(6):
        q = G(lk, rng.standard_normal((1, 3 * D)))
        P = G(lk, [p], np.int64)
        got = m(q, P).numpy()
        want = lk.ops.attention_decode_f32_gpu(q, KC, VC, P, bias, heads).numpy()
        assert np.array_equal(got, want)


def test_runtime_errors(gpu):
    lk = gpu
    ir = """model {
  init {
    return
  }
  exec(%a: tensor<f32[4, 8]>, %b: tensor<f32[9, 4]>) {
    %c = kernel "gemm_f32_gpu_mps"(%a, %b) : tensor<f32[4, 4]>
    return %c
  }
}
"""
    m = lk.compile_ir(ir)
    with pytest.raises(LokinferError, match="gemm"):  # the kernel's own shape check, as a call error
        m(G(lk, np.zeros((4, 8))), G(lk, np.zeros((9, 4))))
    with pytest.raises(LokinferError, match="dim 0"):
        m(G(lk, np.zeros((5, 8))), G(lk, np.zeros((9, 4))))
    with pytest.raises(LokinferError, match="unknown kernel"):
        lk.compile_ir(ir.replace("gemm_f32_gpu_mps", "nope_f32_gpu"))
    with pytest.raises(LokinferError, match="host kernel"):
        lk.compile_ir(ir.replace("gemm_f32_gpu_mps", "gemm_f32_cpu"))


def test_device_error_surfaces_at_a_synchronised_call(gpu):
    lk = gpu
    heads, cap, D = 2, 16, 128
    bias = G(lk, np.zeros(3 * D))

    def step(q, p):
        g = lk.graph.current_graph()
        kc, vc = (g.persistent(lk.TensorType(lk.f32, [cap, D])) for _ in range(2))
        return lk.ops.attention_decode_f32_gpu(q, kc, vc, p, bias, heads)

    m = lk.compile(step, input_types=[lk.TensorType(lk.f32, [1, 3 * D]), lk.TensorType(lk.i64, [1])])
    exe = m._exe
    q = G(lk, rng.standard_normal((1, 3 * D)))
    exe.run([q, G(lk, [3], np.int64)], sync=True)
    with pytest.raises(LokinferError, match="device error 2.*detail 16"):
        exe.run([q, G(lk, [cap], np.int64)], sync=True)
    exe.run([q, G(lk, [4], np.int64)], sync=True)  # the record was cleared
    # the record is per GPU: an error left unread by earlier work is not blamed on a new executable's init
    exe.run([q, G(lk, [cap], np.int64)], sync=False)
    m2 = lk.compile(step, input_types=[lk.TensorType(lk.f32, [1, 3 * D]), lk.TensorType(lk.i64, [1])])
    m2._exe.run([q, G(lk, [5], np.int64)], sync=True)


# ---- bake-init (reference tests/unit/test_compiler.cpp:240-290, tests/python/test_call_api.py:195-220) ---------

BAKE_SRC = """model {
  init {
    return
  }
  exec(%x: tensor<f32[4]>) {
    %w = const.inline dense<[1.0, 2.0, 3.0, 4.0]> : tensor<f32[4]>
    %w2 = kernel "add_f32_gpu"(%w, %w) : tensor<f32[4]>
    %a = kernel "add_f32_gpu"(%x, %w2) : tensor<f32[4]>
    %o = kernel "mul_f32_gpu"(%a, %x) : tensor<f32[4]>
    return %o
  }
}
"""


def test_bake_init_text_model(gpu, tmp_path):
    """2 w is hoisted into init (a kernel on a constant) and baked; the static arena (scratch for %a) is not."""
    lk = gpu
    m = lk.compile_ir(BAKE_SRC)
    x = np.array([0.5, -1.0, 2.0, 3.0], np.float32)
    ref = (x + 2 * np.arange(1, 5, dtype=np.float32)) * x
    X = G(lk, x)
    assert np.array_equal(m(X).numpy(), ref)
    stats = m.bake_init()
    assert stats["baked"] == 1 and stats["baked_bytes"] == 16
    assert stats["init_ops_after"] < stats["init_ops_before"]
    text = m.ir_text()
    assert 'const.internal @"baked' in text
    assert 'kernel "add_f32_gpu"(%w' not in text  # the init kernel is gone
    assert "arena = true" in text                 # scratch memory stays an alloc
    assert np.array_equal(m(X).numpy(), ref)
    # the baked model survives the binary format
    path = tmp_path / "baked.lkm"
    m.save(path)
    back = lk.load(path)
    assert 'const.internal @"baked' in back.ir_text()
    assert np.array_equal(back(X).numpy(), ref)


def test_bake_init_stores_transformed_weights(gpu, tmp_path):
    lk = gpu
    w_np = np.random.default_rng(0).standard_normal((16, 24)).astype(np.float32)
    w = G(lk, w_np)

    def f(x):
        return lk.ops.gemm_f32_gpu(x, lk.ops.transpose_f32_gpu(w))  # the transpose is hoisted into init

    x = G(lk, np.random.default_rng(1).standard_normal((5, 24)))
    model = lk.compile(f, inputs=[x])
    ref = model(x).numpy().copy()
    assert np.abs(ref - x.numpy() @ w_np.T).max() <= 1e-4 * np.abs(ref).max()
    stats = model.bake_init()
    assert stats["baked"] == 1 and stats["baked_bytes"] == 24 * 16 * 4
    assert stats["init_ops_after"] < stats["init_ops_before"]
    ir = model.ir_text()
    assert "transpose_f32_gpu" not in ir and "baked" in ir
    assert 'device = "gpu"' in ir  # resident where the init kernel wrote it
    assert np.array_equal(model(x).numpy(), ref)
    # export: the file holds w^T only (the original w is gone with the init work that read it)
    path = tmp_path / "baked.lkm"
    lk.compile(f, inputs=[x]).save(path, bake_init=True)
    loaded = lk.load(path)
    assert "transpose" not in loaded.ir_text()
    assert np.array_equal(loaded(x).numpy(), ref)
