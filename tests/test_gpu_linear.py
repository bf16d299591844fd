"""The linear layer fused with the loss (``familywise_linear_loss``): logits = hidden @ weight.T
handed over one vocabulary chunk at a time, never as one [N, V] tensor.

Bar: on the same chunk logits (the same ``F.linear`` calls, concatenated on the host), kappa, H and
the per-row losses are bit-identical to the oracle (the definition, reference_impl.py:11-35, with
the strict support of src/cpu/fw_cpu.cpp:96-101), and the support columns are exactly {z > H}.
The gradients of hidden and weight are checked against the oracle's dense logit gradient
multiplied out in fp64 (fp32 inputs: 1e-5 of the largest magnitude; 16-bit inputs, whose results
are rounded to 8 or 11 significant bits: 1e-2), and against the unfused autograd path.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
TOL = {"f32": 1e-5, "bf16": 1e-2, "f16": 1e-2}


def make(dev, N, d, V, dt, seed, spread=3.0):
    rng = np.random.default_rng(seed)
    h = torch.from_numpy(rng.standard_normal((N, d), dtype=np.float32)).to(dev).to(DT[dt])
    w = torch.from_numpy((rng.standard_normal((V, d), dtype=np.float32) * (spread / np.sqrt(d))).astype(np.float32))
    w = w.to(dev).to(DT[dt])
    y = torch.from_numpy(rng.integers(0, V, N).astype(np.int64)).to(dev)
    return h, w, y


def chunk_logits(h, w, chunk):
    """The logits exactly as the fused op sees them: the same F.linear call per chunk."""
    V = w.shape[0]
    return torch.cat([F.linear(h, w[v0:v0 + chunk]) for v0 in range(0, V, chunk)], dim=1)


def dense_grads(z, y, h, w, go_rows):
    """fp64 dhidden and dweight from the oracle's dense logit gradient (scale 1), each row
    multiplied by go_rows."""
    ref = oracle.definition(z, y, scale=1.0)
    g = ref["grad"].astype(np.float64) * go_rows.reshape(-1, 1)
    hn = h.float().cpu().numpy().astype(np.float64)
    wn = w.float().cpu().numpy().astype(np.float64)
    return ref, g @ wn, g.T @ hn


def close(a, ref, tol):
    a = a.float().cpu().numpy().astype(np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(a - ref).max()
    assert err <= tol * scale, f"max error {err:.3e} > {tol:g} x {scale:.3e}"


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("N,d,V,chunk", [(200, 64, 3000, 1000), (130, 72, 5003, 777), (64, 40, 700, 4096),
                                         (1, 16, 33, 1), (257, 128, 20000, 8192)])
def test_forward_parity(dev, dt, N, d, V, chunk):
    import fwloss
    h, w, y = make(dev, N, d, V, dt, seed=N + V)
    res = fwloss.linear_forward(h, w, y, chunk)
    z = chunk_logits(h, w, chunk).float().cpu().numpy()
    yn = y.cpu().numpy()
    ref = oracle.definition(z, yn, scale=1.0, grad=False)
    kappa = res["kappa"].cpu().numpy()
    assert np.array_equal(kappa, ref["kappa"]), np.nonzero(kappa != ref["kappa"])[0][:10]
    assert np.array_equal(res["H"].cpu().numpy().view(np.uint32), ref["H"].view(np.uint32))
    assert np.array_equal(res["losses"].cpu().numpy().view(np.uint32), ref["loss"].view(np.uint32))
    sup = res["support"].cpu().numpy()
    ovf = res["overflow"].cpu().numpy()
    H = ref["H"]
    for r in range(N):
        if ovf[r]:
            continue
        want = np.nonzero(z[r] > H[r])[0]
        assert np.array_equal(np.sort(sup[r, :kappa[r]]), want), f"row {r}"


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_grads(dev, dt, reduction):
    import fwloss
    N, d, V, chunk = 150, 64, 4000, 1024
    h, w, y = make(dev, N, d, V, dt, seed=7)
    hh = h.clone().requires_grad_(True)
    ww = w.clone().requires_grad_(True)
    loss = fwloss.familywise_linear_loss(hh, ww, y, reduction, chunk)
    if reduction == "none":
        go = torch.from_numpy(np.random.default_rng(3).uniform(-2, 2, N).astype(np.float32)).to(dev)
        loss.backward(go.to(loss.dtype))
        go_rows = go.to(loss.dtype).float().cpu().numpy().astype(np.float64)
    else:
        loss.backward()
        go_rows = np.full(N, 1.0 / N if reduction == "mean" else 1.0)
    z = chunk_logits(h, w, chunk).float().cpu().numpy()
    ref, dh_ref, dw_ref = dense_grads(z, y.cpu().numpy(), h, w, go_rows)
    if reduction == "none":   # per-row losses in the logits' dtype
        want = torch.from_numpy(ref["loss"]).to(loss.dtype).float().numpy()
        assert np.array_equal(loss.detach().float().cpu().numpy(), want)
    close(hh.grad, dh_ref, TOL[dt])
    close(ww.grad, dw_ref, TOL[dt])
    assert hh.grad.dtype == h.dtype and ww.grad.dtype == w.dtype


def test_loss_value(dev):
    import fwloss
    h, w, y = make(dev, 300, 64, 6000, "f32", seed=11)
    z = chunk_logits(h, w, 2048).float().cpu().numpy()
    ref = oracle.definition(z, y.cpu().numpy(), scale=1.0, grad=False)
    mean = fwloss.familywise_linear_loss(h, w, y, "mean", 2048)
    total = fwloss.familywise_linear_loss(h, w, y, "sum", 2048)
    none = fwloss.familywise_linear_loss(h, w, y, "none", 2048)
    l64 = ref["loss"].astype(np.float64)
    assert abs(mean.item() - l64.mean()) <= 1e-6 * max(1.0, abs(l64.mean()))
    assert abs(total.item() - l64.sum()) <= 1e-6 * max(1.0, abs(l64.sum()))
    assert np.array_equal(none.cpu().numpy().view(np.uint32), ref["loss"].view(np.uint32))


def test_overflow_rows(dev):
    """Rows with more than the state's capacity of entries near the maximum (here: every logit 0,
    so kappa = V) run on their materialised logits; results are unchanged."""
    import fwloss
    N, d, V, chunk = 40, 32, 3000, 1000
    h, w, y = make(dev, N, d, V, "f32", seed=5)
    h[::7] = 0.0           # these rows: all logits 0
    res = fwloss.linear_forward(h, w, y, chunk)
    ovf = res["overflow"].cpu().numpy()
    assert ovf[::7].all() and not ovf[1::7].any()
    z = chunk_logits(h, w, chunk).float().cpu().numpy()
    yn = y.cpu().numpy()
    ref = oracle.definition(z, yn, scale=1.0, grad=False)
    assert np.array_equal(res["kappa"].cpu().numpy(), ref["kappa"])
    assert (ref["kappa"][::7] == V).all()
    assert np.array_equal(res["H"].cpu().numpy().view(np.uint32), ref["H"].view(np.uint32))
    hh = h.clone().requires_grad_(True)
    ww = w.clone().requires_grad_(True)
    fwloss.familywise_linear_loss(hh, ww, y, "mean", chunk).backward()
    _, dh_ref, dw_ref = dense_grads(z, yn, h, w, np.full(N, 1.0 / N))
    close(hh.grad, dh_ref, 1e-5)
    close(ww.grad, dw_ref, 1e-5)


def test_matches_unfused_autograd(dev):
    """Against familywise_loss on the materialised logits with torch's dense GEMM backward."""
    import fwloss
    N, d, V, chunk = 256, 96, 5000, 5000
    h, w, y = make(dev, N, d, V, "f32", seed=21)
    h1, w1 = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    l1 = fwloss.familywise_linear_loss(h1, w1, y, "mean", chunk)
    l1.backward()
    h2, w2 = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    l2 = fwloss.familywise_loss(F.linear(h2, w2), y, "mean")
    l2.backward()
    assert abs(l1.item() - l2.item()) <= 1e-6 * max(1.0, abs(l2.item()))
    close(h1.grad, h2.grad.double().cpu().numpy(), 1e-5)
    close(w1.grad, w2.grad.double().cpu().numpy(), 1e-5)


def test_label_outside_range(dev):
    """A target outside [0, V) gives loss NaN and no label term, as the fused op does."""
    import fwloss
    N, d, V, chunk = 20, 32, 500, 128
    h, w, y = make(dev, N, d, V, "f32", seed=9)
    y[3] = -1
    y[5] = V
    res = fwloss.linear_forward(h, w, y, chunk)
    z = chunk_logits(h, w, chunk)
    H, losses, _, kappa, _ = fwloss.fw_forward_backward(z, y, 1.0, 1.0)
    assert np.array_equal(res["kappa"].cpu().numpy(), kappa.cpu().numpy())
    assert np.array_equal(res["H"].cpu().numpy().view(np.uint32), H.cpu().numpy().view(np.uint32))
    l = res["losses"].cpu().numpy()
    assert np.isnan(l[3]) and np.isnan(l[5]) and np.isfinite(np.delete(l, [3, 5])).all()
    hh = h.clone().requires_grad_(True)
    fwloss.familywise_linear_loss(hh, w, y, "none", chunk).sum().backward()
    _, _, _, _, g = fwloss.fw_forward_backward(z, y, 1.0, 1.0)   # no label term on rows 3 and 5
    close(hh.grad, (g.double() @ w.double()).cpu().numpy(), 1e-5)


def test_chunk_order_independent(dev):
    """Chunks merged in any order give the same state outcome."""
    import fwloss
    N, d, V, chunk = 100, 48, 3000, 500
    h, w, y = make(dev, N, d, V, "f32", seed=13)
    ext = fwloss._ext
    outs = []
    for order in (range(0, V, chunk), reversed(range(0, V, chunk))):
        st = ext.fw_linear_state(h, N)
        for v0 in order:
            ext.fw_linear_chunk(st, F.linear(h, w[v0:v0 + chunk]), y, v0, V)
        outs.append([t.cpu() for t in ext.fw_linear_finish(st, y, V)[:3]])
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                           b.view(torch.int32) if b.dtype == torch.float32 else b)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_grads_unaligned_hidden_size(dev, dt):
    """d whose rows are not whole 16-byte units: the element-wise gather and scatter paths."""
    import fwloss
    N, d, V, chunk = 90, 37, 2500, 999
    h, w, y = make(dev, N, d, V, dt, seed=17)
    hh = h.clone().requires_grad_(True)
    ww = w.clone().requires_grad_(True)
    fwloss.familywise_linear_loss(hh, ww, y, "sum", chunk).backward()
    z = chunk_logits(h, w, chunk).float().cpu().numpy()
    _, dh_ref, dw_ref = dense_grads(z, y.cpu().numpy(), h, w, np.ones(N))
    close(hh.grad, dh_ref, TOL[dt])
    close(ww.grad, dw_ref, TOL[dt])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("labels", ["one", "zipf"])
@pytest.mark.parametrize("d", [64, 37, 4160])
def test_grads_skewed_labels(dev, dt, labels, d):
    """Columns of weight with many entries (every row labelled with the same column, or Zipf
    labels whose most frequent column takes about a third of the rows): the weight gradient
    splits a long column over the hidden dimension, several wavefronts per column, each output
    still one fma chain over the column's entries in key order (d = 4160 fp32: 17 groups of 64
    units; d = 37: element-wise units)."""
    import fwloss
    N, V, chunk = 600, 3000, 1000
    h, w, y = make(dev, N, d, V, dt, seed=23 + d)
    if labels == "one":
        y = torch.full_like(y, 5)
    else:
        u = np.random.default_rng(d).random(N)
        y = torch.from_numpy(np.minimum(np.floor(u ** -1.2).astype(np.int64) - 1, V - 1)).to(dev)
    print(f"skewed labels {labels} {dt} d={d} max count {int(torch.bincount(y).max())}", flush=True)
    hh = h.clone().requires_grad_(True)
    ww = w.clone().requires_grad_(True)
    fwloss.familywise_linear_loss(hh, ww, y, "sum", chunk).backward()
    z = chunk_logits(h, w, chunk).float().cpu().numpy()
    _, dh_ref, dw_ref = dense_grads(z, y.cpu().numpy(), h, w, np.ones(N))
    close(hh.grad, dh_ref, TOL[dt])
    close(ww.grad, dw_ref, TOL[dt])
    # the same call again gives the same bits (a fixed order of every sum)
    ww2 = w.clone().requires_grad_(True)
    fwloss.familywise_linear_loss(h, ww2, y, "sum", chunk).backward()
    assert torch.equal(ww.grad.view(torch.int16 if ww.grad.element_size() == 2 else torch.int32),
                       ww2.grad.view(torch.int16 if ww2.grad.element_size() == 2 else torch.int32))


def test_only_hidden_needs_grad(dev):
    import fwloss
    N, d, V, chunk = 64, 32, 1000, 300
    h, w, y = make(dev, N, d, V, "f32", seed=19)
    hh = h.clone().requires_grad_(True)
    fwloss.familywise_linear_loss(hh, w, y, "mean", chunk).backward()
    z = chunk_logits(h, w, chunk).float().cpu().numpy()
    _, dh_ref, _ = dense_grads(z, y.cpu().numpy(), h, w, np.full(N, 1.0 / N))
    close(hh.grad, dh_ref, 1e-5)
    assert w.grad is None


@pytest.mark.parametrize("spread", [0.5, 3.0, 12.0])
def test_lm_head_scale_against_unfused(dev, spread):
    """An LM-head shape (4096 tokens, d = 512, V = 50000, bf16) at flat, moderate and peaky logit
    spreads, against the unfused layer + familywise_loss with autograd's dense backward: the same
    loss (to the fp32 sum order) and gradients within bf16 rounding."""
    import fwloss
    N, d, V, chunk = 4096, 512, 50000, 8192
    g = torch.Generator(device=dev).manual_seed(int(spread * 10))
    h = torch.randn(N, d, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, d, device=dev, generator=g) * (spread / d ** 0.5)).to(torch.bfloat16)
    y = torch.randint(0, V, (N,), device=dev, generator=g)
    print(f"lm head spread={spread}", flush=True)
    h1, w1 = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    l1 = fwloss.familywise_linear_loss(h1, w1, y, "mean", chunk)
    l1.backward()
    res = fwloss.linear_forward(h, w, y, chunk)
    z = chunk_logits(h, w, chunk)
    H, losses, _, kappa, _ = fwloss.fw_forward_backward(z, y)
    assert torch.equal(res["kappa"], kappa)
    assert torch.equal(res["H"].view(torch.int32), H.view(torch.int32))
    assert torch.equal(res["losses"].view(torch.int32), losses.view(torch.int32))
    h2, w2 = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    l2 = fwloss.familywise_loss(torch.cat([F.linear(h2, w2[v0:v0 + chunk]) for v0 in range(0, V, chunk)], 1), y)
    l2.backward()
    assert abs(l1.float().item() - l2.float().item()) <= 1e-2 * max(1.0, abs(l2.float().item()))
    close(h1.grad, h2.grad.double().cpu().numpy(), 2e-2)
    close(w1.grad, w2.grad.double().cpu().numpy(), 2e-2)


def test_backward_graph_capture(dev):
    """The layer's backward (fw_linear_grads) holds no host synchronisation: captured in a HIP
    graph and replayed, with eager work and synchronisations between the replays, every replay
    gives the eager gradients bit for bit (the key array is sized for every row's largest count;
    the entries' count stays on the device)."""
    import fwloss
    ext = fwloss._ext
    N = 300
    h, w, y = make(dev, N, 64, 5000, "f32", seed=11)
    res = fwloss.linear_forward(h, w, y, chunk=1000)
    assert res["dense"] is None
    rs = torch.full((1,), 1.0 / N, device=dev)
    args = (h, w, y, res["kappa_sparse"], res["support"], rs, True, True)
    dh0, dw0 = ext.fw_linear_grads(*args)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            ext.fw_linear_grads(*args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dh, dw = ext.fw_linear_grads(*args)
    for i in range(3):
        a = torch.randn(512, 512, device=dev)
        (a @ a).sum().item()
        g.replay()
        torch.cuda.synchronize()
        print(f"replay {i}", flush=True)
        assert torch.equal(dh, dh0) and torch.equal(dw, dw0), f"replay {i} differs from the eager gradients"
