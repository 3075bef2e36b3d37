"""rg_linear, the decode-step projection kernel, against a float32 reference on the CPU.

out = x . weight^T with bf16 / f16 operands: the kernel accumulates in fp32 and rounds each
output once, so it must equal the fp32 product of the same rounded operands within one
rounding of the output type (plus the fp32 reordering, far smaller).  Shapes: the Llama-3.2-1B
decode projections at 128 rows (qkv, o_proj, gate/up, down) and edge cases — rows not a
multiple of 16, a single row, the smallest K (one 128-wide chunk, shorter than the copy ring),
row-strided x and out, workgroup shapes of 4, 2 and 1 n-blocks and 1 to 8 row blocks, row tiles
with a partial last tile, and column-tile counts that are and are not multiples of 8 (the
XCD-aware and the plain tile order).
"""
from __future__ import annotations

import pytest
import torch

from railgun_amd import _lib
from railgun_amd.ops import RailgunError, linear, linear_residual, linear_workspace_bytes

pytestmark = pytest.mark.gpu

TORCH = {"bf16": torch.bfloat16, "f16": torch.float16}


def _check(out: torch.Tensor, x: torch.Tensor, w: torch.Tensor, what: str, ref_on_device: bool = False) -> None:
    # (the float32 product of the largest shapes runs on the device: torch's fp32 GEMM there is
    # a plain fp32 product, no reduced-precision inputs)
    ref = (x.float() @ w.float().T).cpu() if ref_on_device else x.float().cpu() @ w.float().cpu().T
    got = out.float().cpu()
    # one rounding of the output type (2^-8 relative for bf16, 2^-11 for f16), on a floor of the
    # typical magnitude for outputs near zero
    rtol = 2 ** -8 if out.dtype == torch.bfloat16 else 2 ** -11
    err = (got - ref).abs()
    bound = rtol * ref.abs() + 1e-3 * ref.abs().mean() + 1e-6
    assert bool((err <= bound).all()), f"{what}: max excess {float((err - bound).max()):.3g}"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M,N,K", [(128, 3072, 2048), (128, 2048, 2048), (128, 16384, 2048), (128, 2048, 8192),
                                   (1, 16, 128), (7, 48, 256), (33, 4096, 128), (100, 8192, 384), (16, 2064, 512),
                                   (1, 16384, 2048), (64, 128256, 256), (128, 192, 2048), (100, 8192, 2048),
                                   (77, 1040, 1024)])
def test_linear_matches_fp32(device, M, N, K, dt):
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).to(TORCH[dt]).to(device)
    w = (0.02 * torch.randn(N, K, generator=g)).to(TORCH[dt]).to(device)
    out = linear(x, w)
    torch.cuda.synchronize()
    _check(out, x, w, f"{M}x{N}x{K} {dt}")
    again = linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), out.view(torch.int16)), "not deterministic"


@pytest.mark.parametrize("M,N,K,dt", [(128, 128256, 2048, "bf16"), (100, 128256, 2048, "f16"), (17, 128256, 2048, "bf16"),
                                      (37, 65536, 128, "bf16"), (90, 131072, 128, "f16"), (64, 128256, 256, "f16"),
                                      (33, 32768, 256, "bf16"), (65, 32768, 384, "f16"), (16, 32768, 256, "bf16"),
                                      (17, 32768, 384, "f16")])
def test_linear_large_n(device, M, N, K, dt):
    """Large N: the Llama LM head (N = 128,256) at 128, 100 and 17 rows (full, ragged and
    two-block row tiles), N = 64 k / 128 k with K of one chunk, fp16; the wide form's edges (17,
    33 and 65 rows: the first row counts of its 32-, 64- and 128-row X tiles; 16 rows: the skinny
    form); against the fp32 product and repeatable bit for bit."""
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(TORCH[dt]).to(device)
    w = (0.02 * torch.randn(N, K, generator=g)).to(TORCH[dt]).to(device)
    out = linear(x, w)
    torch.cuda.synchronize()
    _check(out, x, w, f"{M}x{N}x{K} {dt}", ref_on_device=True)
    again = linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), out.view(torch.int16)), "not deterministic"


def test_linear_large_n_strided_and_residual(device):
    """Large N with x a column slice of a wider activation and out a column slice of a wider
    buffer (untouched around it), and the residual epilogue at a large N: bit for bit the
    rounded product added to the residual and rounded (the residual add of rg_rms_norm)."""
    g = torch.Generator().manual_seed(11)
    K, N, M = 1024, 32768, 128
    act = torch.randn(M, K + 64, generator=g).to(torch.bfloat16).to(device)
    x = act[:, 64:]
    w = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).to(device)
    buf = torch.full((M, N + 32), 7.0, dtype=torch.bfloat16, device=device)
    out = buf[:, 16:16 + N]
    linear(x, w, out)
    torch.cuda.synchronize()
    _check(out, x, w, "strided, large N", ref_on_device=True)
    assert bool((buf[:, :16] == 7.0).all()) and bool((buf[:, 16 + N:] == 7.0).all())
    M2, N2, K2 = 48, 65536, 640
    x2 = torch.randn(M2, K2, generator=g).to(torch.bfloat16).to(device)
    w2 = (0.02 * torch.randn(N2, K2, generator=g)).to(torch.bfloat16).to(device)
    res = torch.randn(M2, N2, generator=g).to(torch.bfloat16).to(device)
    prod = linear(x2, w2)  # the same tiles, rounded once
    want = (res.float() + prod.float()).to(torch.bfloat16)
    linear_residual(x2, w2, res)
    torch.cuda.synchronize()
    _check(prod, x2, w2, "large N", ref_on_device=True)
    assert torch.equal(res.view(torch.int16), want.view(torch.int16)), "residual epilogue"


def test_linear_strided_rows(device):
    """x a column slice of a wider activation and out a column slice of a wider buffer."""
    g = torch.Generator().manual_seed(3)
    wide = torch.randn(37, 2048 + 64, generator=g).to(torch.bfloat16).to(device)
    x = wide[:, 64:]                                   # row stride 2112
    w = (0.02 * torch.randn(512, 2048, generator=g)).to(torch.bfloat16).to(device)
    buf = torch.full((37, 512 + 32), 7.0, dtype=torch.bfloat16, device=device)
    out = buf[:, 16:16 + 512]
    linear(x, w, out)
    torch.cuda.synchronize()
    _check(out, x, w, "strided")
    assert bool((buf[:, :16] == 7.0).all()) and bool((buf[:, 16 + 512:] == 7.0).all()), "wrote outside out"


def test_linear_refuses_unsupported_shapes(device):
    w = torch.zeros(32, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(RailgunError) as e:
        linear(torch.zeros(129, 64, dtype=torch.bfloat16, device=device), w)   # more rows than a decode batch
    assert e.value.code == _lib.RG_ERR_NOT_SUPPORTED
    with pytest.raises(RailgunError):
        linear(torch.zeros(4, 96, dtype=torch.bfloat16, device=device),
               torch.zeros(32, 96, dtype=torch.bfloat16, device=device))     # K not a multiple of 128


@pytest.mark.parametrize("M,N,K", [(128, 2048, 8192), (1, 2048, 8192), (64, 2048, 8192), (8, 512, 8192),
                                   (16, 2048, 16384)])
def test_linear_split_k(device, M, N, K):
    """Narrow / deep layers split K over workgroups into an fp32 workspace and a fixed-order
    reduce; the split result, the unsplit one (no workspace) and fp32 all agree, and repeated
    split calls are bit-identical."""
    from railgun_amd.ops import linear_workspace_bytes
    ws_bytes = linear_workspace_bytes(M, N, K)
    assert ws_bytes > 0, "deep, narrow layers split K on a 256-CU device"
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(device)
    w = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).to(device)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device=device)   # NaN-filled: every partial is written
    split = linear(x, w, workspace=ws)
    again = linear(x, w, workspace=ws)
    unsplit = linear(x, w, workspace=torch.empty(16, dtype=torch.uint8, device=device))  # too small: one pass
    torch.cuda.synchronize()
    _check(split, x, w, f"split {M}x{N}x{K}")
    _check(unsplit, x, w, f"unsplit {M}x{N}x{K}")
    assert torch.equal(again.view(torch.int16), split.view(torch.int16)), "split K not deterministic"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M,I,K", [(128, 8192, 2048), (1, 8192, 2048), (37, 512, 256), (100, 1040, 1024)])
def test_linear_silu_mul(device, M, I, K, dt):
    """The gate/up projection with SiLU·mul in the epilogue against the fp32 products rounded the
    way rg_linear + rg_silu_and_mul round them: g, u to the activation dtype, silu(g) rounded,
    then the product."""
    from railgun_amd.ops import interleave_gate_up, linear_silu_mul
    g = torch.Generator().manual_seed(M + I + K)
    x = torch.randn(M, K, generator=g).to(TORCH[dt]).to(device)
    w = (0.05 * torch.randn(2 * I, K, generator=g)).to(TORCH[dt]).to(device)
    got = linear_silu_mul(x, interleave_gate_up(w))
    again = linear_silu_mul(x, interleave_gate_up(w))
    torch.cuda.synchronize()
    t = TORCH[dt]
    xf, wf = x.float().cpu(), w.float().cpu()
    gv = (xf @ wf[:I].T).to(t).float()
    uv = (xf @ wf[I:].T).to(t).float()
    act = (gv / (1 + torch.exp(-gv))).to(t).float()
    ref = (act * uv).to(t).float()
    err = (got.float().cpu() - ref).abs()
    # First-order propagation of one ulp in g and in u (the GEMM's fp32 sums taken in another
    # order can round either way) and of the roundings of silu(g) and of the product:
    # |d out| <= eps (|u| |silu'(g)| |g| + 2 |silu(g)| |u| + |out|), eps one ulp relative.
    eps = 2 ** -7 if dt == "bf16" else 2 ** -10
    sig = torch.sigmoid(gv)
    dsilu = (sig * (1 + gv * (1 - sig))).abs()
    bound = eps * (uv.abs() * dsilu * gv.abs() + 2 * act.abs() * uv.abs() + ref.abs()) + 1e-3 * ref.abs().mean() + 1e-6
    assert bool((err <= bound).all()), f"max excess {float((err - bound).max()):.3g}"
    assert torch.equal(again.view(torch.int16), got.view(torch.int16)), "not deterministic"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("T,H,Hkv,D,K,bs", [(128, 32, 8, 64, 2048, 16), (1, 32, 8, 64, 2048, 16),
                                            (37, 8, 2, 32, 256, 32), (100, 4, 4, 64, 384, 16)])
def test_linear_qkv_rope_reshape_and_cache(device, kernels, T, H, Hkv, D, K, bs, dt):
    """The q/k/v projection with RoPE and the paged-cache write in its epilogue against the
    unfused path (rg_linear without split, then rg_qkv_rope_reshape_and_cache on its output).
    Both round q/k/v to the activation dtype before the rotation and rotate with the same
    unfused arithmetic; they differ only where the fp32 sums, taken in another order, round
    q/k/v to the other neighbour: one ulp of the pre-rotation value times |cos| + |sin|, plus
    one ulp of the result.  Slots of padding tokens (-1) and every other slot stay untouched."""
    from railgun_amd.ops import linear, rope_cos_sin_table
    t = TORCH[dt]
    g = torch.Generator().manual_seed(T * 31 + D + K)
    x = torch.randn(T, K, generator=g).to(t).to(device)
    w = (0.05 * torch.randn((H + 2 * Hkv) * D, K, generator=g)).to(t).to(device)
    nb = max(8, 2 * T // bs + 2)
    pos = torch.randint(0, 500, (T,), generator=g, dtype=torch.int32).to(device)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    if T > 3:
        slots[3] = -1
    slots = slots.to(device)
    cs = rope_cos_sin_table(512, D, 500000.0, device)
    pool_a = torch.randn(nb, 2, Hkv, bs, D, generator=g).to(t).to(device)
    pool_b = pool_a.clone()
    q_a = torch.empty(T, H, D, dtype=t, device=device)
    q_b = torch.empty(T, H, D, dtype=t, device=device)
    kernels.launch_linear_qkv_rope_reshape_and_cache(x, w, q_a, pool_a[:, 0], pool_a[:, 1], cs, pos, slots,
                                                     H, Hkv, D, bs)
    qkv = linear(x, w, workspace=torch.empty(16, dtype=torch.uint8, device=device))
    kernels.launch_qkv_rope_reshape_and_cache(qkv, q_b, pool_b[:, 0], pool_b[:, 1], cs, pos, slots, H, Hkv, D, bs, T)
    again = torch.empty_like(q_a)
    kernels.launch_linear_qkv_rope_reshape_and_cache(x, w, again, pool_a[:, 0], pool_a[:, 1], cs, pos, slots,
                                                     H, Hkv, D, bs)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), q_a.view(torch.int16)), "not deterministic"

    eps = 2 ** -7 if dt == "bf16" else 2 ** -10
    half = D // 2
    csc = cs.cpu()[pos.cpu().long()]                                     # [T, 2 half]: cos | sin
    trig = (csc[:, :half].abs() + csc[:, half:].abs()).repeat(1, 2)      # |cos| + |sin| per column
    pre = (x.float().cpu() @ w.float().cpu().T).view(T, H + 2 * Hkv, D)
    pre_mag = torch.cat([pre[..., :half], pre[..., half:]], -1).abs()
    pair = torch.maximum(pre_mag, torch.cat([pre_mag[..., half:], pre_mag[..., :half]], -1))

    def bound(ref, heads, rotated, rows):
        if rotated:
            extra = pair[rows][:, heads] * trig[rows][:, None, :]
        else:
            extra = pre[rows][:, heads].abs()
        return eps * (ref.abs() + extra) + 1e-6

    every = torch.arange(T)
    qa, qb = q_a.float().cpu(), q_b.float().cpu()
    assert bool(((qa - qb).abs() <= bound(qb, slice(0, H), True, every)).all()), \
        f"q: max diff {float((qa - qb).abs().max()):.3g}"
    pa, pb = pool_a.float().cpu(), pool_b.float().cpu()
    sl = slots.cpu().long()
    written = torch.zeros(nb * bs, dtype=torch.bool)
    written[sl[sl >= 0]] = True
    flat_a = pa.permute(0, 3, 1, 2, 4).reshape(nb * bs, 2, Hkv, D)   # [slot, k/v, head, D]
    flat_b = pb.permute(0, 3, 1, 2, 4).reshape(nb * bs, 2, Hkv, D)
    assert torch.equal(flat_a[~written], flat_b[~written]), "wrote a slot outside the mapping"
    tok = torch.nonzero(sl >= 0).squeeze(1)
    for kv, heads, rot in ((0, slice(H, H + Hkv), True), (1, slice(H + Hkv, H + 2 * Hkv), False)):
        got, ref = flat_a[sl[tok], kv], flat_b[sl[tok], kv]
        assert bool(((got - ref).abs() <= bound(ref, heads, rot, tok)).all()), \
            f"{'kv'[kv]} cache: max diff {float((got - ref).abs().max()):.3g}"


def test_linear_qkv_rope_refuses_unsupported(device, kernels):
    """Head dims other than 32 / 64 and more than 128 tokens are refused, not mis-computed."""
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=device)
    w = torch.zeros(4 * 128, 256, dtype=torch.bfloat16, device=device)
    q = torch.empty(4, 2, 128, dtype=torch.bfloat16, device=device)
    pool = torch.zeros(4, 2, 1, 16, 128, dtype=torch.bfloat16, device=device)
    cs = torch.zeros(16, 128, dtype=torch.float32, device=device)
    i = torch.zeros(4, dtype=torch.int32, device=device)
    with pytest.raises(RailgunError) as e:
        kernels.launch_linear_qkv_rope_reshape_and_cache(x, w, q, pool[:, 0], pool[:, 1], cs, i, i, 2, 1, 128, 16)
    assert e.value.code == _lib.RG_ERR_NOT_SUPPORTED
    # Shapes that disagree with the head counts are refused on the host before any launch: the
    # entry would read (H + 2 H_kv) D weight rows and write T H D values of q.
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=device)
    q = torch.empty(4, 2, 64, dtype=torch.bfloat16, device=device)
    pool = torch.zeros(4, 2, 1, 16, 64, dtype=torch.bfloat16, device=device)
    cs = torch.zeros(16, 64, dtype=torch.float32, device=device)
    good_w = torch.zeros(4 * 64, 256, dtype=torch.bfloat16, device=device)
    bad = [dict(w=torch.zeros(3 * 64, 256, dtype=torch.bfloat16, device=device)),   # too few weight rows
           dict(w=torch.zeros(4 * 64, 384, dtype=torch.bfloat16, device=device)),   # K of the weight != x's
           dict(q=torch.empty(4, 1, 64, dtype=torch.bfloat16, device=device)),       # q_out too small
           dict(cs=torch.zeros(16, 32, dtype=torch.float32, device=device))]         # cos/sin rows too narrow
    for case in bad:
        with pytest.raises(RailgunError) as e:
            kernels.launch_linear_qkv_rope_reshape_and_cache(x, case.get("w", good_w), case.get("q", q), pool[:, 0],
                                                             pool[:, 1], case.get("cs", cs), i, i, 2, 1, 64, 16)
        assert e.value.code == _lib.RG_ERR_INVALID_ARGUMENT, case


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M,N,K", [(128, 2048, 2048), (128, 2048, 8192), (37, 512, 256), (1, 2048, 8192)])
def test_linear_residual(device, M, N, K, dt):
    """residual += x @ W^T equals rg_linear's rounded output added to the residual and rounded
    (the residual add of rg_rms_norm) bit for bit, with and without a split of K; the residual
    a column slice of a wider buffer whose other columns stay untouched."""
    t = TORCH[dt]
    g = torch.Generator().manual_seed(M + N + 3 * K)
    x = torch.randn(M, K, generator=g).to(t).to(device)
    w = (0.02 * torch.randn(N, K, generator=g)).to(t).to(device)
    buf = torch.randn(M, N + 24, generator=g).to(t).to(device)
    res = buf[:, 8:8 + N]                               # row stride N + 24
    before = buf.clone()
    ws = torch.empty(max(16, linear_workspace_bytes(M, N, K)), dtype=torch.uint8, device=device)
    linear_residual(x, w, res, workspace=ws)
    delta = linear(x, w, workspace=ws)
    torch.cuda.synchronize()
    want = (before[:, 8:8 + N].float() + delta.float()).to(t)
    assert torch.equal(res.view(torch.int16), want.view(torch.int16))
    assert torch.equal(buf[:, :8].view(torch.int16), before[:, :8].view(torch.int16))
    assert torch.equal(buf[:, 8 + N:].view(torch.int16), before[:, 8 + N:].view(torch.int16))


def _norm_ref(x, nw, eps):
    """fp32 RmsNorm of x (without rounding) and the row scales."""
    xf = x.float().cpu()
    rs = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return xf * rs * nw.float().cpu(), rs


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M,I,K", [(128, 8192, 2048), (1, 8192, 2048), (37, 512, 256), (100, 1040, 1024),
                                   (5, 1024, 8192), (64, 2048, 4096)])
def test_rms_norm_linear_silu_mul(device, M, I, K, dt):
    """The MLP input RmsNorm folded into the gate/up projection with SiLU·mul, against the fp32
    chain.  The kernel feeds round(x w_norm) to the MFMA and scales the sums by 1 / rms(x); the
    bound carries one rounding of every operand product (|x w_norm| |W| summed, times the row
    scale) and of g and u, then SiLU·mul to first order, and the two output roundings."""
    from railgun_amd.ops import interleave_gate_up, linear_silu_mul
    t = TORCH[dt]
    g = torch.Generator().manual_seed(M + I + K + 1)
    x = (3 * torch.randn(M, K, generator=g)).to(t).to(device)
    nw = (1 + 0.2 * torch.randn(K, generator=g)).to(t).to(device)
    w = (0.05 * torch.randn(2 * I, K, generator=g)).to(t).to(device)
    eps = 1e-5
    got = linear_silu_mul(x, interleave_gate_up(w), norm_weight=nw, eps=eps)
    again = linear_silu_mul(x, interleave_gate_up(w), norm_weight=nw, eps=eps)
    torch.cuda.synchronize()
    h, rs = _norm_ref(x, nw, eps)
    wf = w.float().cpu()
    gv, uv = h @ wf[:I].T, h @ wf[I:].T
    absx = (x.float().cpu() * nw.float().cpu()).abs()
    e = 2 ** -8 if dt == "bf16" else 2 ** -11
    dg = e * rs * (absx @ wf[:I].abs().T) + e * gv.abs()
    du = e * rs * (absx @ wf[I:].abs().T) + e * uv.abs()
    sig = torch.sigmoid(gv)
    act = gv * sig
    ref = act * uv
    dsilu = (sig * (1 + gv * (1 - sig))).abs()
    bound = 2 * (dsilu * dg * uv.abs() + act.abs() * du + 2 * e * ref.abs()) + 1e-3 * ref.abs().mean() + 1e-6
    err = (got.float().cpu() - ref).abs()
    assert bool((err <= bound).all()), f"max excess {float((err - bound).max()):.3g}"
    assert torch.equal(again.view(torch.int16), got.view(torch.int16)), "not deterministic"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("T,H,Hkv,D,K,bs", [(128, 32, 8, 64, 2048, 16), (1, 32, 8, 64, 2048, 16),
                                            (37, 8, 2, 32, 256, 32), (9, 16, 4, 64, 8192, 16)])
def test_rms_norm_linear_qkv_rope_reshape_and_cache(device, kernels, T, H, Hkv, D, K, bs, dt):
    """The attention input RmsNorm folded into the q/k/v projection with RoPE and the cache
    write, against the fp32 chain (bound as in the MLP test: one rounding of every operand
    product and of q/k/v, carried through the rotation by |cos| + |sin|, plus the output
    rounding).  Slots outside the mapping stay untouched."""
    from railgun_amd.ops import rope_cos_sin_table
    tt = TORCH[dt]
    g = torch.Generator().manual_seed(T * 13 + D + K)
    x = (3 * torch.randn(T, K, generator=g)).to(tt).to(device)
    nw = (1 + 0.2 * torch.randn(K, generator=g)).to(tt).to(device)
    w = (0.05 * torch.randn((H + 2 * Hkv) * D, K, generator=g)).to(tt).to(device)
    nb = max(8, 2 * T // bs + 2)
    pos = torch.randint(0, 500, (T,), generator=g, dtype=torch.int32).to(device)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    if T > 3:
        slots[3] = -1
    slots = slots.to(device)
    cs = rope_cos_sin_table(512, D, 500000.0, device)
    pool = torch.randn(nb, 2, Hkv, bs, D, generator=g).to(tt).to(device)
    before = pool.clone()
    q = torch.empty(T, H, D, dtype=tt, device=device)
    eps = 1e-5
    kernels.launch_linear_qkv_rope_reshape_and_cache(x, w, q, pool[:, 0], pool[:, 1], cs, pos, slots, H, Hkv, D, bs,
                                                     norm_weight=nw, eps=eps)
    torch.cuda.synchronize()
    h, rs = _norm_ref(x, nw, eps)
    wf = w.float().cpu()
    pre = (h @ wf.T).view(T, H + 2 * Hkv, D)
    absx = (x.float().cpu() * nw.float().cpu()).abs()
    e = 2 ** -8 if dt == "bf16" else 2 ** -11
    dpre = (e * rs * (absx @ wf.abs().T)).view(T, H + 2 * Hkv, D) + e * pre.abs()
    half = D // 2
    csc = cs.cpu()[pos.cpu().long()]
    c, s = csc[:, :half][:, None, :], csc[:, half:][:, None, :]
    lo, hi = pre[..., :half], pre[..., half:]
    rot = torch.cat([lo * c - hi * s, hi * c + lo * s], -1)
    dl, dh = dpre[..., :half], dpre[..., half:]
    drot = torch.cat([dl * c.abs() + dh * s.abs(), dh * c.abs() + dl * s.abs()], -1)
    bound = 2 * (drot + e * rot.abs()) + 1e-5
    got_q = q.float().cpu()
    assert bool(((got_q - rot[:, :H]).abs() <= bound[:, :H]).all()), \
        f"q: max excess {float(((got_q - rot[:, :H]).abs() - bound[:, :H]).max()):.3g}"
    sl = slots.cpu().long()
    flat = pool.float().cpu().permute(0, 3, 1, 2, 4).reshape(nb * bs, 2, Hkv, D)
    flat0 = before.float().cpu().permute(0, 3, 1, 2, 4).reshape(nb * bs, 2, Hkv, D)
    written = torch.zeros(nb * bs, dtype=torch.bool)
    written[sl[sl >= 0]] = True
    assert torch.equal(flat[~written], flat0[~written]), "wrote a slot outside the mapping"
    tok = torch.nonzero(sl >= 0).squeeze(1)
    kref, kb = rot[tok, H:H + Hkv], bound[tok, H:H + Hkv]
    vref = pre[tok, H + Hkv:]
    vb = 2 * (dpre[tok, H + Hkv:] + e * vref.abs()) + 1e-5
    assert bool(((flat[sl[tok], 0] - kref).abs() <= kb).all()), "k cache"
    assert bool(((flat[sl[tok], 1] - vref).abs() <= vb).all()), "v cache"


@pytest.mark.parametrize("M", [1, 4, 128])
def test_rms_norm_linear_fp16_residual_range(device, kernels, M):
    """fp16 residual rows far from 1 in size, through both folded norms: |x| up to 3e4 with
    norm weights up to 3 (x * w_norm past fp16's 65504 if it were rounded before the division
    by rms(x), which the unfused chain does first) and |x| around 1e-4 (x * w_norm in fp16's
    subnormals).  The outputs are finite and within the fp32 chain's bound of one rounding of
    every W * w_norm product, of the projection and of the outputs."""
    from railgun_amd.ops import interleave_gate_up, linear_silu_mul, rope_cos_sin_table
    t = torch.float16
    g = torch.Generator().manual_seed(77 + M)
    K, I = 2048, 512
    mags = torch.tensor([3e4, 1e-4, 1.0, 2e4])[torch.arange(M) % 4]
    x = (mags[:, None] * torch.randn(M, K, generator=g).clamp(-2, 2)).to(t)
    nw = (1 + 2 * torch.rand(K, generator=g)).to(t)
    assert float((x.float() * nw.float()).abs().max()) > 65504 and bool(torch.isfinite(x.float()).all())
    w = (0.05 * torch.randn(2 * I, K, generator=g)).to(t)
    x, nw, w = x.to(device), nw.to(device), w.to(device)
    eps = 1e-5
    e = 2 ** -11
    h, rs = _norm_ref(x, nw, eps)
    wf = w.float().cpu()
    absx = (x.float().cpu() * nw.float().cpu()).abs()

    got = linear_silu_mul(x, interleave_gate_up(w), norm_weight=nw, eps=eps).float().cpu()
    gv, uv = h @ wf[:I].T, h @ wf[I:].T
    dg = e * rs * (absx @ wf[:I].abs().T) + e * gv.abs()
    du = e * rs * (absx @ wf[I:].abs().T) + e * uv.abs()
    sig = torch.sigmoid(gv)
    act, ref = gv * sig, gv * sig * uv
    dsilu = (sig * (1 + gv * (1 - sig))).abs()
    bound = 2 * (dsilu * dg * uv.abs() + act.abs() * du + 2 * e * ref.abs()) + 1e-3 * ref.abs().mean() + 1e-6
    assert bool(torch.isfinite(got).all()), "gate/up: non-finite output"
    assert bool(((got - ref).abs() <= bound).all()), f"gate/up: max excess {float(((got - ref).abs() - bound).max()):.3g}"

    H, Hkv, D, bs = 8, 2, 64, 16
    wq = (0.05 * torch.randn((H + 2 * Hkv) * D, K, generator=g)).to(t).to(device)
    nb = M // bs + 4
    pos = torch.arange(M, dtype=torch.int32, device=device)
    slots = torch.arange(M, dtype=torch.int32, device=device)
    cs = rope_cos_sin_table(max(M, 2), D, 500000.0, device)
    pool = torch.zeros(nb, 2, Hkv, bs, D, dtype=t, device=device)
    q = torch.empty(M, H, D, dtype=t, device=device)
    kernels.launch_linear_qkv_rope_reshape_and_cache(x, wq, q, pool[:, 0], pool[:, 1], cs, pos, slots, H, Hkv, D, bs,
                                                     norm_weight=nw, eps=eps)
    torch.cuda.synchronize()
    wqf = wq.float().cpu()
    pre = (h @ wqf.T).view(M, H + 2 * Hkv, D)
    dpre = (e * rs * (absx @ wqf.abs().T)).view(M, H + 2 * Hkv, D) + e * pre.abs()
    half = D // 2
    csc = cs.cpu()[pos.cpu().long()]
    c, s = csc[:, :half][:, None, :], csc[:, half:][:, None, :]
    lo, hi = pre[..., :half], pre[..., half:]
    rot = torch.cat([lo * c - hi * s, hi * c + lo * s], -1)
    dl, dh = dpre[..., :half], dpre[..., half:]
    drot = torch.cat([dl * c.abs() + dh * s.abs(), dh * c.abs() + dl * s.abs()], -1)
    qb = 2 * (drot + e * rot.abs()) + 1e-5
    got_q = q.float().cpu()
    assert bool(torch.isfinite(got_q).all()), "q: non-finite output"
    assert bool(((got_q - rot[:, :H]).abs() <= qb[:, :H]).all()), \
        f"q: max excess {float(((got_q - rot[:, :H]).abs() - qb[:, :H]).max()):.3g}"
    flat = pool.float().cpu().permute(0, 3, 1, 2, 4).reshape(nb * bs, 2, Hkv, D)[:M]
    assert bool(torch.isfinite(flat).all()), "cache: non-finite rows"
    assert bool(((flat[:, 0] - rot[:, H:H + Hkv]).abs() <= qb[:, H:H + Hkv]).all()), "k cache"


def test_rms_norm_linear_refuses_unsupported(device, kernels):
    """in_features past the LDS copy of the norm weight, a misaligned norm weight and a
    negative eps are refused."""
    from railgun_amd.ops import linear_silu_mul
    x = torch.zeros(4, 8192 + 128, dtype=torch.bfloat16, device=device)
    w = torch.zeros(64, 8192 + 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(RailgunError) as e:
        linear_silu_mul(x, w, norm_weight=torch.ones(8192 + 128, dtype=torch.bfloat16, device=device), eps=1e-5)
    assert e.value.code == _lib.RG_ERR_NOT_SUPPORTED
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=device)
    w = torch.zeros(64, 256, dtype=torch.bfloat16, device=device)
    nw = torch.ones(257, dtype=torch.bfloat16, device=device)[1:]       # 2 bytes past 16-byte alignment
    with pytest.raises(RailgunError):
        linear_silu_mul(x, w, norm_weight=nw, eps=1e-5)
    with pytest.raises(RailgunError):
        linear_silu_mul(x, w, norm_weight=torch.ones(256, dtype=torch.bfloat16, device=device), eps=-1.0)
