"""The Backend activation and training ops on the GPU, through the C ABI.

Parity with the oracle's restatement of crates/cpu (oracle/oracle.c):
* add_bias, bias_grad, sgd_step, convert and mse_grad's dy: bit for bit (each formula is
  evaluated as written, one rounding per operation; bias_grad sums rows in order);
* mse_grad's loss: the order of summation is the backend's (crates/core/src/lib.rs:98-101), so
  it is checked against the sequential sum with the bound n*u*sum(d*d)/n and against f64
  within the reference's 1e-6 (crates/cpu/src/training.rs:143-176), and for determinism;
* gelu and gelu_backward: the same f32 expression as the reference with the device's expf,
  so within |err| <= 4e-7 * max(1, |x|) (times |dy| for the derivative) of the oracle, and
  within the reference's 1e-6 of the normal-cdf definition (invariants.rs:462-500).
The pipeline test restates crates/pipeline's single-rank training step on its own fixture
(crates/pipeline/tests/pipeline.rs:17-37) through the HIP backend only.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from helpers import rng
from linalg_hip import backend as B
from test_training_oracle import SAMPLES, gelu_prime_ref, gelu_ref, pattern

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hb():
    backend = B.HipBackend(0)
    yield backend
    backend.close()


def f32(v):
    return np.asarray(v, dtype=np.float32)


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def up(hb, a, shape=None):
    a = f32(a)
    return hb.upload_f32(list(shape if shape is not None else a.shape), a.ravel())


def same_storage(t: B.Tensor, **kw) -> B.Tensor:
    f = dict(storage=t.storage, dtype=t.dtype, shape=list(t.shape), strides=list(t.strides),
             offset=t.offset)
    f.update(kw)
    return B.Tensor(**f)


def test_every_v2_method_known_answers(hb):
    # crates/cpu/src/training.rs:72-91.
    x = up(hb, [[1, 2, 3], [4, 5, 6]])
    b = up(hb, [0.5, -0.5, 1.0])
    y = hb.alloc(B.DType.F32, [2, 3])
    db = hb.alloc(B.DType.F32, [3])
    t = up(hb, np.zeros((2, 3)))
    dy = hb.alloc(B.DType.F32, [2, 3])
    w = up(hb, [1.0, 1.0, 1.0])
    h = hb.alloc(B.DType.BF16, [2, 3])
    start = len(hb.debug_launches())
    hb.add_bias(x, b, y)
    hb.bias_grad(y, db)
    loss = hb.mse_grad(y, t, dy)
    hb.sgd_step(w, db, 0.5)
    hb.convert(y, h)
    hb.convert(h, x)
    assert hb.download_f32(x).tolist() == [1.5, 1.5, 4.0, 4.5, 4.5, 7.0]
    assert hb.download_f32(db).tolist() == [0.0, 0.0, 0.0]
    assert hb.download_f32(w).tolist() == [1.0 - 0.5 * 6.0, 1.0 - 0.5 * 6.0, 1.0 - 0.5 * 11.0]
    assert loss > 0.0
    assert hb.debug_launches()[start:] == ["add_bias_f32", "bias_grad_f32", "mse_grad_f32",
                                           "sgd_step_f32", "convert_f32_bf16", "convert_bf16_f32"]


@pytest.mark.parametrize("rows,cols", [(7, 33), (8, 64), (1, 1), (300, 1024), (5, 4097)])
def test_add_bias_is_bit_exact_and_runs_in_place(hb, rows, cols):
    xs, bs = pattern(rows * cols, 1).reshape(rows, cols), pattern(cols, 2)
    want = oracle.add_bias(xs, bs)
    x, b = up(hb, xs), up(hb, bs)
    y = hb.alloc(B.DType.F32, [rows, cols])
    hb.add_bias(x, b, y)
    assert np.array_equal(bits(hb.download_f32(y)), bits(want.ravel()))
    hb.add_bias(x, b, same_storage(x))
    assert np.array_equal(bits(hb.download_f32(x)), bits(want.ravel()))


@pytest.mark.parametrize("rows,cols", [(64, 37), (1000, 513), (4099, 130), (3, 5000), (17, 1)])
def test_bias_grad_is_the_sequential_column_sum(hb, rows, cols):
    ds, seed = pattern(rows * cols, 3).reshape(rows, cols), pattern(cols, 4)
    want = oracle.bias_grad(ds, seed)
    dpre, db = up(hb, ds), up(hb, seed)
    hb.bias_grad(dpre, db)
    assert np.array_equal(bits(hb.download_f32(db)), bits(want))
    # B = 0 leaves db unchanged and launches nothing.
    n0 = len(hb.debug_launches())
    hb.bias_grad(hb.alloc(B.DType.F32, [0, cols]), db)
    assert np.array_equal(bits(hb.download_f32(db)), bits(want))
    assert len(hb.debug_launches()) == n0


@pytest.mark.parametrize("shape", [(8, 65), (1, 1), (3, 5), (1024, 1024), (4097, 33),
                                   (2049, 2052), (2049, 2051)])
def test_mse_grad(hb, shape):
    n = int(np.prod(shape))
    g = rng(n)
    ys = g.uniform(-1, 1, n).astype(np.float32).reshape(shape)
    ts = g.uniform(-1, 1, n).astype(np.float32).reshape(shape)
    want_dy, want_loss = oracle.mse_grad(ys, ts)
    y, t = up(hb, ys), up(hb, ts)
    dy = hb.alloc(B.DType.F32, list(shape))
    loss = hb.mse_grad(y, t, dy)
    assert np.array_equal(bits(hb.download_f32(dy)), bits(want_dy.ravel()))
    d = ys.astype(np.float64) - ts.astype(np.float64)
    sq = float((d * d).sum())
    # Any fixed summation order: within (n + 1) u of the sum of squares, over n.
    assert abs(loss - float(want_loss)) <= (n + 2) * 2.0 ** -24 * sq / n + 1e-30
    if n <= 520:
        assert abs(loss - sq / n) <= 1e-6
    # Deterministic, in place (dy = y) and with y sharing target's storage.
    loss2 = hb.mse_grad(y, t, same_storage(y))
    assert np.float32(loss2) == np.float32(loss)
    assert np.array_equal(bits(hb.download_f32(y)), bits(want_dy.ravel()))
    zeros = hb.alloc(B.DType.F32, list(shape))
    assert hb.mse_grad(t, same_storage(t), zeros) == 0.0
    assert not bits(hb.download_f32(zeros)).any()


@pytest.mark.parametrize("n", [300, 1, 7, 1 << 20])
def test_sgd_step_updates_and_zeroes(hb, n):
    ws, gs = pattern(n, 7), pattern(n, 8)
    lr = np.float32(1e-3)
    want_w, _ = oracle.sgd_step(ws, gs, lr)
    w, dw = up(hb, ws), up(hb, gs)
    hb.sgd_step(w, dw, float(lr))
    assert np.array_equal(bits(hb.download_f32(w)), bits(want_w))
    assert not bits(hb.download_f32(dw)).any()


def test_convert_matches_the_reference_rounding_and_is_exact_back(hb):
    specials = np.asarray([0x00000000, 0x80000000, 0x3F800000, 0x3F808000, 0x3F818000, 0x3F808001,
                           0x3F807FFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F7FFF, 0x7F800000, 0xFF800000,
                           0x00010000, 0x80018000, 0x00000001, 0x7F800001, 0xFF800001, 0x7FC00000,
                           0xFFFFFFFF, 0x7F812345], np.uint32).view(np.float32)
    g = rng(9)
    randoms = g.uniform(-1e4, 1e4, 4093).astype(np.float32)
    raw = g.integers(0, 2 ** 32, 4096, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for cases in (specials, randoms, raw):
        x = hb.upload(B.DType.F32, [cases.size], cases.tobytes())
        h = hb.alloc(B.DType.BF16, [cases.size])
        hb.convert(x, h)
        got = np.frombuffer(hb.download(h), dtype=np.uint16)
        assert np.array_equal(got, oracle.f32_to_bf16(cases))
    allh = np.arange(65536, dtype=np.uint16)
    hsrc = hb.upload(B.DType.BF16, [65536], allh.tobytes())
    back = hb.alloc(B.DType.F32, [65536])
    hb.convert(hsrc, back)
    assert np.array_equal(bits(hb.download_f32(back)), allh.astype(np.uint32) << 16)


def gelu_tolerance(x):
    return 4e-7 * np.maximum(1.0, np.abs(x.astype(np.float64)))


def test_gelu_and_backward_on_the_reference_samples(hb):
    x = f32(SAMPLES)
    y = hb.alloc(B.DType.F32, [x.size])
    hb.gelu(up(hb, x), y)
    got = hb.download_f32(y)
    for gv, s in zip(got, x):
        assert abs(float(gv) - gelu_ref(float(s))) <= 1e-6, s
    assert np.all(np.abs(got.astype(np.float64) - oracle.gelu(x)) <= gelu_tolerance(x))
    dyv = f32([s * 0.5 - 0.25 for s in SAMPLES])
    dx = hb.alloc(B.DType.F32, [x.size])
    hb.gelu_backward(up(hb, x), up(hb, dyv), dx)
    got = hb.download_f32(dx)
    for gv, s, d in zip(got, x, dyv):
        assert abs(float(gv) - float(d) * gelu_prime_ref(float(s))) <= 1e-6, s


@pytest.mark.parametrize("n", [1 << 20, 4097])
def test_gelu_and_backward_against_the_oracle(hb, n):
    g = rng(n + 3)
    x = (g.standard_normal(n) * 3.0).astype(np.float32)
    dyv = g.uniform(-1, 1, n).astype(np.float32)
    y = hb.alloc(B.DType.F32, [n])
    xt = up(hb, x)
    hb.gelu(xt, y)
    got = hb.download_f32(y)
    want = oracle.gelu(x)
    assert np.all(np.abs(got.astype(np.float64) - want) <= gelu_tolerance(x))
    exact = float(np.mean(bits(got) == bits(want)))
    assert exact > 0.5, f"only {exact:.3f} of GELU outputs match the reference bits"
    dx = hb.alloc(B.DType.F32, [n])
    hb.gelu_backward(xt, up(hb, dyv), dx)
    got = hb.download_f32(dx)
    want = oracle.gelu_backward(x, dyv)
    tol = gelu_tolerance(x) * np.maximum(np.abs(dyv), 1e-30) + 1e-30
    assert np.all(np.abs(got.astype(np.float64) - want) <= tol)
    # In place: y = GELU(y).
    hb.gelu(xt, same_storage(xt))
    assert np.array_equal(bits(hb.download_f32(xt)), bits(hb.download_f32(y)))


def test_errors_change_nothing_and_launch_nothing(hb):
    seed = pattern(6, 13)
    x = up(hb, pattern(6, 11), [2, 3])
    b = up(hb, pattern(3, 12))
    y = up(hb, seed, [2, 3])
    odd = same_storage(y, strides=[1, 2])
    hbf = hb.alloc(B.DType.BF16, [3])
    h = hb.alloc(B.DType.BF16, [2, 3])
    start = hb.debug_launches()
    calls = [
        (lambda: hb.add_bias(x, same_storage(y, shape=[3], strides=[1]), y), "Alias"),
        (lambda: hb.add_bias(x, b, odd), "UnsupportedLayout"),
        (lambda: hb.bias_grad(x, same_storage(x, shape=[3], strides=[1])), "Alias"),
        (lambda: hb.mse_grad(x, y, same_storage(y)), "Alias"),
        (lambda: hb.mse_grad(x, x, odd), "UnsupportedLayout"),
        (lambda: hb.sgd_step(y, same_storage(y), 0.1), "Alias"),
        (lambda: hb.convert(h, same_storage(y, dtype=B.DType.BF16)), "Dtype"),
        (lambda: hb.convert(x, same_storage(x, dtype=B.DType.BF16)), "Alias"),
        (lambda: hb.gelu(hb.alloc(B.DType.F16, [2, 3]), y), "Dtype"),
        (lambda: hb.gelu(x, odd), "UnsupportedLayout"),
        (lambda: hb.gelu_backward(x, hbf, y), "Dtype"),
    ]
    for call, kind in calls:
        with pytest.raises(B.BackendError) as e:
            call()
        assert e.value.kind == kind
    assert np.array_equal(bits(hb.download_f32(y)), bits(seed))
    assert hb.debug_launches() == start


# ---- crates/pipeline/tests/pipeline.rs: one rank, three layers, two microbatches ----------
WIDTHS = [3, 4, 2, 3]
X0 = [0.5, -1.0, 0.25, 1.0, 0.0, -0.5]
X1 = [-0.25, 0.5, 1.0, 0.0, -1.0, 0.25]
DY0 = [0.1, -0.2, 0.3, 0.0, 0.25, -0.1]
DY1 = [-0.3, 0.1, 0.0, 0.2, -0.2, 0.4]


def weight(layer: int) -> np.ndarray:
    rows, cols = WIDTHS[layer], WIDTHS[layer + 1]
    r = np.arange(rows, dtype=np.float32)[:, None]
    c = np.arange(cols, dtype=np.float32)[None, :]
    return (np.float32(0.1) * (r + np.float32(1.0)) - np.float32(0.05) * (c + np.float32(1.0))
            + np.float32(0.02) * np.float32(layer)).astype(np.float32)


def seq_gemm(a, b, c=None, beta=0.0):
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), np.float32) if c is None else c.copy()
    oracle.gemm_seq(m, n, k, 1.0, beta, np.ascontiguousarray(a), 0, [k, 1],
                    np.ascontiguousarray(b), 0, [n, 1], out.reshape(-1), 0, [n, 1])
    return out


def cpu_train(xs, dys, weights):
    """pipeline::train on one rank (crates/pipeline/src/lib.rs:149-229), with the crates/cpu
    restatement for every op."""
    dw = [np.zeros_like(w) for w in weights]
    ys = []
    for x, dy in zip(xs, dys):  # one stage: F(m) then B(m)
        pre, act = [], []
        cur = x
        for w in weights:
            p = seq_gemm(cur, w)
            a = oracle.gelu(p)
            pre.append(p)
            act.append(a)
            cur = a
        ys.append(act[-1])
        g = dy
        for l in range(len(weights) - 1, -1, -1):
            dpre = oracle.gelu_backward(pre[l], g)
            inp = x if l == 0 else act[l - 1]
            dw[l] = seq_gemm(np.ascontiguousarray(inp.T), dpre, dw[l], beta=1.0)
            g = seq_gemm(dpre, np.ascontiguousarray(weights[l].T))
    return ys, dw


def hip_train(hb, xs, dys, weights):
    """The same step through HipBackend: every op is one lg_backend_* call."""
    w_t = [up(hb, w) for w in weights]
    dw = [hb.alloc(B.DType.F32, list(w.shape)) for w in weights]
    ys = []
    for x, dy in zip(xs, dys):
        x_t, dy_t = up(hb, x), up(hb, dy)
        batch = x.shape[0]
        pre, act = [], []
        cur = x_t
        for w in w_t:
            p = hb.alloc(B.DType.F32, [batch, w.shape[1]])
            hb.gemm(cur, w, p, 1.0, 0.0)
            a = hb.alloc(B.DType.F32, [batch, w.shape[1]])
            hb.gelu(p, a)
            pre.append(p)
            act.append(a)
            cur = a
        ys.append(act[-1])
        g = dy_t
        for l in range(len(w_t) - 1, -1, -1):
            k, n = w_t[l].shape
            dpre = hb.alloc(B.DType.F32, [batch, n])
            hb.gelu_backward(pre[l], g, dpre)
            inp = x_t if l == 0 else act[l - 1]
            hb.gemm(B.transpose_matrix(inp), dpre, dw[l], 1.0, 1.0)
            dx = hb.alloc(B.DType.F32, [batch, k])
            hb.gemm(dpre, B.transpose_matrix(w_t[l]), dx, 1.0, 0.0)
            g = dx
    return [hb.download_f32(y).reshape(-1) for y in ys], [hb.download_f32(d) for d in dw]


def test_single_rank_pipeline_step_matches_the_cpu_restatement(hb):
    xs = [f32(X0).reshape(2, 3), f32(X1).reshape(2, 3)]
    dys = [f32(DY0).reshape(2, 3), f32(DY1).reshape(2, 3)]
    weights = [weight(l) for l in range(3)]
    ry, rdw = cpu_train(xs, dys, weights)
    gy, gdw = hip_train(hb, xs, dys, weights)
    for got, want in zip(gy, ry):
        assert np.max(np.abs(got - want.ravel())) <= 1e-6
    for got, want in zip(gdw, rdw):
        assert np.max(np.abs(got - want.ravel())) <= 1e-6


def test_pipeline_step_at_a_larger_width(hb):
    # Two layers of width 256 -> 384 -> 128, batch 192: the kernels' tiled paths.
    g = rng(77)
    widths = [256, 384, 128]
    weights = [(g.standard_normal((widths[i], widths[i + 1])) * 0.05).astype(np.float32)
               for i in range(2)]
    xs = [(g.standard_normal((192, 256)) * 0.5).astype(np.float32) for _ in range(2)]
    dys = [(g.standard_normal((192, 128)) * 0.1).astype(np.float32) for _ in range(2)]
    ry, rdw = cpu_train(xs, dys, weights)
    gy, gdw = hip_train(hb, xs, dys, weights)
    for got, want in zip(gy, ry):
        assert np.max(np.abs(got - want.ravel())) <= 1e-5 * max(1.0, float(np.max(np.abs(want))))
    for got, want in zip(gdw, rdw):
        assert np.max(np.abs(got - want.ravel())) <= 1e-5 * max(1.0, float(np.max(np.abs(want))))
