"""GPU parity of the whole cached-KV query (tabicl_mi355_query: column blocks over the cached
inducing-point K|V, row interactor, cached ICL blocks, decoder; the reference's _make_query_fn,
scripts/tabicl_tpu_bucketed.py:768-834) against a CPU restatement in float64.

The restatement is written here from the same call sites, with the oracle's attention: feature grouping
by explicit index loops, the in-linear with the skip rule, each layer's LayerNorm / GEMMs / GELU in
float64, `pk_cross_ref` for the column and CLS attention, `pk_self_ref` with the oracle's RoPE tables
for the row attention, and for the ICL stage the rounding points of the bf16 path (as in
test_gpu_icl_stage.py) around `splash_sdpa_ref`. Each stage is compared on the GPU's input to that
stage, so errors do not compound across stages; `cached_query` itself is checked bit for bit against the
stages run one after the other.

Bars (written here): column and row stages in fp32 (the reference's precision for them): max abs error
<= 1e-4 x max(1, max |ref|) (the residual stream reaches a few units) and <= 1e-3 x max |ref| over the
non-skip columns; in bf16: max abs error <= 5e-2 x max |ref| (each GEMM output is a bf16 value, three
blocks deep). Logits (bf16 ICL stage):
max abs error <= 2e-2 x max(1, max |ref|). Shapes: 2 estimators, 64 test rows, 100 features with 100 and
97 real (the row stage's key mask and the grouping's wrap-around), 3 column blocks over 128 cached
inducing keys, 3 row blocks (104 tokens: the persistent row kernel in bf16), 2 ICL blocks over 900 of
1000 cached train rows, 10 classes.
"""
import pytest
import torch

from parity import check
from query_ref import C, E, ICLH, NI, SKIP, Rope, as_f64, column_ref, icl_ref, model, row_ref, to_device

pytestmark = pytest.mark.gpu
B, T, NF = 2, 64, 100


def _stage_check(out, ref, dtype, what):
    # fp32: 1e-4 of the residual stream's scale (max(1, max|ref|), values reach a few units three blocks
    # deep) and 1e-3 x max|ref|; bf16: 5e-2 x max|ref|
    scale = max(1.0, float(ref.abs().max()))
    if dtype == torch.float32:
        check(out, ref, torch.float32, what, abs_tol=1e-4 * scale)
    else:
        check(out, ref, dtype, what, abs_tol=5e-2 * scale, rel_tol=5e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32_col_row", "bf16_col_row"])
def test_cached_query_matches_restatement(dev, dtype):
    import tabicl_mi355_icl as icl
    import tabicl_mi355_query as Q
    w, g = model(dtype)
    wd = to_device(w, dev)
    rope = Rope()
    X = torch.randn(B, T, NF, generator=g)
    d = torch.tensor([NF, NF - 3])
    hidden = [torch.randn(B, NF + C, NI, E, generator=g).to(dtype) for _ in range(3)]
    col_cache = Q.ColumnKVCache(3, B, NF + C, NI, E, dtype, dev)
    for b in range(3):
        col_cache.append_projected(b, hidden[b].to(dev), wd.column.blocks[b])
    cap, train = 1000, 900
    icl_cache = icl.IclKVCache(B, 2, ICLH, cap, 64, torch.bfloat16, dev)
    kc = torch.randn(B, 2, ICLH, cap, 64, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, 2, ICLH, cap, 64, generator=g).to(torch.bfloat16)
    for b in range(2):
        icl_cache.append(b, kc[:, b].to(dev), vc[:, b].to(dev))
    valid = torch.tensor([train], dtype=torch.int32, device=dev)
    Xd, dd = X.to(dev), d.to(dev)
    print(f"[query] composed cached query, column/row {dtype}", flush=True)
    with torch.no_grad():
        src = Q.column_stage(Xd, dd, col_cache, wd.column)
        reprs = Q.row_stage(src, dd, wd.row, rope)
        x = icl_cache.query_blocks(reprs.float(), wd.icl_blocks, valid)
        logits = Q.decode(x, wd.decoder)
        whole = Q.cached_query(Xd, dd, col_cache, icl_cache, wd, valid, rope)
    torch.cuda.synchronize()
    assert torch.equal(whole, logits)
    assert logits.shape == (B, T, 10) and torch.isfinite(logits).all()
    # column stage: the K|V cache as the GPU wrote it (a GEMM output) is the restatement's input
    w64 = as_f64(w)
    kvc = col_cache.kv.double().cpu()
    ref_src = column_ref(X, d, kvc, w64.column)
    live = slice(C, None)  # the reserved slots hold the skip value exactly on both sides
    assert torch.equal(src[:, :C].float().cpu(), torch.full_like(src[:, :C].float().cpu(), SKIP))
    _stage_check(src[:, live], ref_src[:, live], dtype, "column stage")
    # row stage on the GPU's column output
    ref_reprs = row_ref(src.double().cpu(), d, w64.row, rope)
    _stage_check(reprs, ref_reprs, dtype, "row stage")
    # ICL stage + decoder on the GPU's row representation
    ref_logits = icl_ref(reprs.cpu(), w.icl_blocks, kc, vc, train, w.decoder)
    tol = 2e-2 * max(1.0, float(ref_logits.abs().max()))
    check(logits, ref_logits, torch.bfloat16, "logits", abs_tol=tol, rel_tol=1.0)
