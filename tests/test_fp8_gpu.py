"""The fp8 (e4m3) KV pool on the GPU: quantising slot-write and dequantising decode.

The slot-write is bit-exact against the oracle's quantiser (oracle/fp8.py,
pinned against torch's float8_e4m3fn). Attention over an fp8 pool is held to
the bf16 bar (max-abs 2e-2, mean-abs 2e-3) against the fp64 oracle over the
same dequantised rows; beside that, how far the quantised cache moves the
answer from the bf16 cache on the same unquantised K/V is bounded (the
reference's planned "tolerance parity test against fp16/bf16",
docs/roadmap.md section 2.5).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.paged_kernels import kv_scatter, paged_decode
from oracle import fp8
from oracle.attention import attend
from tests.helpers import PagedBatch, assert_within, to_numpy

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
FP8 = torch.float8_e4m3fn


def _codes(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def _to_pool(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes)).to(DEV).view(FP8)


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layout", ["bhtd", "bthd", "strided_dim"])
@pytest.mark.parametrize(("k_scale", "v_scale"), [(1.0, 1.0), (0.25, 3.0)])
def test_quantising_slot_write_is_bit_exact(src_dtype, layout, k_scale, v_scale):
    g = torch.Generator(device=DEV).manual_seed(3)
    batch, heads, tokens, dim, num_slots = 3, 8, 5, 128, 97
    shape = (batch, tokens, heads, dim) if layout == "bthd" else (batch, heads, tokens, dim)
    k = (torch.randn(shape, generator=g, device=DEV) * 30).to(src_dtype)   # some values saturate
    v = (torch.randn(shape, generator=g, device=DEV) * 30).to(src_dtype)
    if layout == "bthd":
        k, v = k.transpose(1, 2), v.transpose(1, 2)
    if layout == "strided_dim":
        k = torch.cat([k, k], dim=3)[..., ::2]
        v = torch.cat([v, v], dim=3)[..., ::2]
    before = torch.randint(0, 255, (num_slots, heads, dim), generator=g, device=DEV, dtype=torch.uint8)
    before[before == 0x7F] = 0  # no NaN codes, so equality below is plain
    kp, vp = before.clone().view(FP8), before.clone().view(FP8)
    slots = torch.tensor([[5, 96, 0, 41, 17, 8, 60, 3, 77, 12, 30, 90, 2, 55, -1]], device=DEV)
    slots[0, -1] = 1000  # out of range: skipped
    kv_scatter(kp, vp, slots, k, v, k_scale=k_scale, v_scale=v_scale)

    want_k, want_v = _codes(before), _codes(before)
    kf = to_numpy(k).astype(np.float32)
    vf = to_numpy(v).astype(np.float32)
    for i, s in enumerate(slots[0].tolist()):
        if not 0 <= s < num_slots:
            continue
        b, t = divmod(i, tokens)
        want_k[s] = fp8.quantize(kf[b, :, t, :], k_scale)
        want_v[s] = fp8.quantize(vf[b, :, t, :], v_scale)
    assert np.array_equal(_codes(kp), want_k)
    assert np.array_equal(_codes(vp), want_v)


def _fp8_batch(context_lens, k_scale, v_scale, q_dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, seed=0,
               num_slots=65536, width=None):
    """A decode batch whose pools are quantised by the oracle; returns it, the fp8 pools and the fp64 oracle."""
    b = PagedBatch(context_lens, dtype=q_dtype, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=128,
                   num_slots=num_slots, seed=seed, width=width)
    kc = fp8.quantize(to_numpy(b.key_pool), k_scale)
    vc = fp8.quantize(to_numpy(b.value_pool), v_scale)
    kd, vd = fp8.dequantize(kc, k_scale), fp8.dequantize(vc, v_scale)
    want = attend(to_numpy(b.query), kd, vd, b.slot_table.cpu().numpy(), np.asarray(context_lens), b.scaling,
                  b.groups, dtype=np.float64)
    return b, _to_pool(kc), _to_pool(vc), want


@pytest.mark.parametrize("kernel", ["auto", "equal_splits"])
@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("k_scale", "v_scale"), [(1.0, 1.0), (0.05, 0.2)])
def test_fp8_decode_matches_the_oracle_over_dequantised_rows(kernel, q_dtype, k_scale, v_scale):
    ctx = [1, 31, 32, 33, 500, 1023, 2100, 4096]
    b, kp, vp, want = _fp8_batch(ctx, k_scale, v_scale, q_dtype=q_dtype, seed=4)
    out = paged_decode(b.query, kp, vp, b.slot_table, b.context_lens_t, b.scaling, b.groups, num_splits=4,
                       kernel=kernel, k_scale=k_scale, v_scale=v_scale)
    assert_within(out, want / 1.0, 2e-2, 2e-3)


@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(32, 8), (8, 8), (16, 1), (20, 4)])
def test_fp8_decode_groupings(num_heads, num_kv_heads):
    b, kp, vp, want = _fp8_batch([7, 300, 1500], 0.5, 0.5, num_heads=num_heads, num_kv_heads=num_kv_heads, seed=5,
                                 num_slots=8192)
    out = paged_decode(b.query, kp, vp, b.slot_table, b.context_lens_t, b.scaling, b.groups, k_scale=0.5,
                       v_scale=0.5)
    assert_within(out, want, 2e-2, 2e-3)


@pytest.mark.parametrize("width", [None, 4096])
@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(32, 8), (16, 1), (20, 4)])
def test_fp8_short_contexts(num_heads, num_kv_heads, width):
    """Contexts of at most 1,000 keys in a table as wide as the longest (the short kernel: one
    work-group per sequence and KV head) and in a wide one (the balanced split)."""
    b, kp, vp, want = _fp8_batch([1, 33, 300, 1000], 0.5, 0.25, num_heads=num_heads, num_kv_heads=num_kv_heads,
                                 seed=6, num_slots=8192, width=width)
    out = paged_decode(b.query, kp, vp, b.slot_table, b.context_lens_t, b.scaling, b.groups, k_scale=0.5,
                       v_scale=0.25)
    assert_within(out, want, 2e-2, 2e-3)


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16])
def test_fp8_decode_queries_of_any_scale(q_dtype):
    """The fp8 scores take the query as e4m3 terms after a power-of-two scale per head: heads
    at 2^-20 .. 2^12 of the usual size, an all-zero head, and rows whose elements spread over
    16 binades all meet the bar."""
    b, kp, vp, _ = _fp8_batch([5, 64, 700, 2049], 0.5, 0.25, q_dtype=q_dtype, seed=9, num_slots=8192)
    g = torch.Generator(device="cpu").manual_seed(3)
    q = b.query.float().cpu()
    spread = torch.pow(2.0, -torch.randint(0, 17, q.shape, generator=g).float())
    q[:, 1::4] *= spread[:, 1::4]
    head_scale = torch.tensor([2.0 ** -20, 1.0, 2.0 ** -6, 2.0 ** 5] * (q.shape[1] // 4))
    if q_dtype == torch.bfloat16:
        head_scale[3::8] = 2.0 ** 12
    q *= head_scale.view(1, -1, 1)
    q[:, 2] = 0.0
    b.query = q.to(q_dtype).to(DEV)
    kd = fp8.dequantize(_codes(kp), 0.5)
    vd = fp8.dequantize(_codes(vp), 0.25)
    want = attend(to_numpy(b.query), kd, vd, b.slot_table.cpu().numpy(), np.asarray(b.context_lens), b.scaling,
                  b.groups, dtype=np.float64)
    out = paged_decode(b.query, kp, vp, b.slot_table, b.context_lens_t, b.scaling, b.groups, k_scale=0.5,
                       v_scale=0.25)
    assert_within(out, want, 2e-2, 2e-3)


def test_c2_fp8_pool_full_size_and_against_the_bf16_cache():
    """Config 2's decode step on an fp8 pool: at the bf16 bar against the oracle over the
    dequantised rows, and within a bounded distance of the same step on the bf16 pool."""
    from liteinfer_amd.workloads import decode_step

    step = decode_step("c2", seed=0)
    kp = torch.empty(step.key_pool.shape, dtype=FP8, device=DEV)
    vp = torch.empty_like(kp)
    all_slots = torch.arange(kp.shape[0], device=DEV).view(1, -1)
    kv_scatter(kp, vp, all_slots, step.key_pool.unsqueeze(0).transpose(1, 2),
               step.value_pool.unsqueeze(0).transpose(1, 2))
    g = step.geometry
    out8 = paged_decode(step.query, kp, vp, step.slot_table, step.context_lens, g.scaling, g.groups)
    out16 = paged_decode(step.query, step.key_pool, step.value_pool, step.slot_table, step.context_lens,
                         g.scaling, g.groups)
    kd = fp8.dequantize(_codes(kp), 1.0)
    vd = fp8.dequantize(_codes(vp), 1.0)
    want = attend(to_numpy(step.query), kd, vd, step.slot_table.cpu().numpy(),
                  np.asarray(step.host_context_lens), g.scaling, g.groups, dtype=np.float32)
    assert_within(out8, want, 2e-2, 2e-3)
    diff = (out8.float() - out16.float()).abs()
    assert diff.max().item() <= 2e-2 and diff.mean().item() <= 2e-3, (diff.max().item(), diff.mean().item())


def test_fp8_pool_rejects_what_it_cannot_serve():
    b = PagedBatch([40], dtype=torch.float32, num_heads=8, num_kv_heads=2, head_dim=128, num_slots=256)
    kp = torch.zeros(256, 2, 128, dtype=FP8, device=DEV)
    with pytest.raises(ValueError, match="bfloat16 or float16"):
        paged_decode(b.query, kp, kp.clone(), b.slot_table, b.context_lens_t, b.scaling, b.groups)
    q = b.query.to(torch.bfloat16)
    with pytest.raises(ValueError, match="k_scale"):
        paged_decode(q, kp, kp.clone(), b.slot_table, b.context_lens_t, b.scaling, b.groups, k_scale=0.0)
    kp64 = torch.zeros(256, 2, 64, dtype=FP8, device=DEV)
    b64 = PagedBatch([40], dtype=torch.bfloat16, num_heads=8, num_kv_heads=2, head_dim=64, num_slots=256)
    with pytest.raises(ValueError, match="MFMA kernel only"):
        paged_decode(b64.query, kp64, kp64.clone(), b64.slot_table, b64.context_lens_t, b64.scaling, b64.groups)


def _fp8_packed(context_lens, query_lens, k_scale, v_scale, q_dtype=torch.bfloat16, num_heads=32, num_kv_heads=8,
                seed=0, num_slots=32768):
    b = PagedBatch(context_lens, query_lens, dtype=q_dtype, num_heads=num_heads, num_kv_heads=num_kv_heads,
                   head_dim=128, num_slots=num_slots, seed=seed)
    kc = fp8.quantize(to_numpy(b.key_pool), k_scale)
    vc = fp8.quantize(to_numpy(b.value_pool), v_scale)
    qsl = to_numpy(b.query_start_loc).astype(np.int32)
    want = attend(to_numpy(b.query), fp8.dequantize(kc, k_scale), fp8.dequantize(vc, v_scale),
                  b.slot_table.cpu().numpy(), np.asarray(context_lens), b.scaling, b.groups, query_start_loc=qsl,
                  dtype=np.float64)
    return b, _to_pool(kc), _to_pool(vc), want


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("k_scale", "v_scale"), [(1.0, 1.0), (0.05, 0.2)])
@pytest.mark.parametrize("one_query_rows", [None, False])
def test_fp8_prefill_matches_the_oracle_over_dequantised_rows(q_dtype, k_scale, v_scale, one_query_rows):
    """Chunks over prefixes and alone, straddling stage boundaries, beside one-query rows."""
    from liteinfer_amd.paged_kernels import paged_prefill

    ctx = [1, 40, 300, 129, 64, 700, 1500]
    q = [1, 33, 200, 1, 64, 31, 257]
    b, kp, vp, want = _fp8_packed(ctx, q, k_scale, v_scale, q_dtype=q_dtype, seed=7)
    out = paged_prefill(b.query, kp, vp, b.slot_table, b.context_lens_t, b.query_start_loc, max(q), b.scaling,
                        b.groups, one_query_rows=one_query_rows, k_scale=k_scale, v_scale=v_scale)
    assert_within(out, want, 2e-2, 2e-3)


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("one_query_rows", [None, False])
def test_fp8_prefill_queries_of_any_scale(q_dtype, one_query_rows):
    """The prefill's fp8 scores take each query row as e4m3 terms after its own power-of-two
    scale: rows at 2^-20 .. 2^12 of the usual size, all-zero rows and rows whose elements
    spread over 16 binades, in chunks and one-query rows, all meet the bar."""
    from liteinfer_amd.paged_kernels import paged_prefill

    ctx = [300, 1, 129, 700, 64]
    q = [200, 1, 1, 31, 64]
    b, kp, vp, _ = _fp8_packed(ctx, q, 0.5, 0.25, q_dtype=q_dtype, seed=11)
    g = torch.Generator(device="cpu").manual_seed(5)
    x = b.query.float().cpu()
    spread = torch.pow(2.0, -torch.randint(0, 17, x.shape, generator=g).float())
    x[:, 1::4] *= spread[:, 1::4]
    head_scale = torch.tensor([2.0 ** -20, 1.0, 2.0 ** -6, 2.0 ** 5] * (x.shape[1] // 4))
    if q_dtype == torch.bfloat16:
        head_scale[3::8] = 2.0 ** 12
    x *= head_scale.view(1, -1, 1)
    x[:, 2] = 0.0
    b.query = x.to(q_dtype).to(DEV)
    qsl = to_numpy(b.query_start_loc).astype(np.int32)
    want = attend(to_numpy(b.query), fp8.dequantize(_codes(kp), 0.5), fp8.dequantize(_codes(vp), 0.25),
                  b.slot_table.cpu().numpy(), np.asarray(ctx), b.scaling, b.groups, query_start_loc=qsl,
                  dtype=np.float64)
    out = paged_prefill(b.query, kp, vp, b.slot_table, b.context_lens_t, b.query_start_loc, max(q), b.scaling,
                        b.groups, one_query_rows=one_query_rows, k_scale=0.5, v_scale=0.25)
    assert_within(out, want, 2e-2, 2e-3)


_MANY_ROWS = np.random.default_rng(13).integers(200, 3000, size=120).tolist()


@pytest.mark.parametrize(
    ("ctx", "q"),
    [([700] + _MANY_ROWS, [300] + [1] * len(_MANY_ROWS)), ([30000, 45000, 600, 2600], [1, 1, 512, 1])],
    ids=["rows-outweigh-one-chunk", "long-rows-in-pieces"],
)
def test_fp8_rows_and_chunks_share_the_prefill_launch(ctx, q):
    """fp8 pools: the one-query rows run as the decode split in the lockstep
    prefill launch's first work-groups, which then join the chunks."""
    from liteinfer_amd.paged_kernels import paged_prefill

    b, kp, vp, want = _fp8_packed(ctx, q, 0.05, 0.2, seed=9)
    out = paged_prefill(b.query, kp, vp, b.slot_table, b.context_lens_t, b.query_start_loc, max(q), b.scaling,
                        b.groups, k_scale=0.05, v_scale=0.2)
    assert_within(out, want, 2e-2, 2e-3)


@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(8, 8), (16, 1), (32, 16)])
def test_fp8_prefill_groupings(num_heads, num_kv_heads):
    from liteinfer_amd.paged_kernels import paged_prefill

    ctx, q = [90, 5000, 33], [90, 130, 1]
    b, kp, vp, want = _fp8_packed(ctx, q, 0.5, 2.0, num_heads=num_heads, num_kv_heads=num_kv_heads, seed=8)
    out = paged_prefill(b.query, kp, vp, b.slot_table, b.context_lens_t, b.query_start_loc, max(q), b.scaling,
                        b.groups, k_scale=0.5, v_scale=2.0)
    assert_within(out, want, 2e-2, 2e-3)


def test_cache_layer_fp8_pool_end_to_end():
    """BlockPool(cache_quant="fp8") through KVCache payloads and the `paged` boundary: the
    same answer as the dense eager kernel reading the same fp8 pool (which dequantises)."""
    from liteinfer_amd.attention import eager_attention, paged_attention
    from liteinfer_amd.cache.block_pool import BlockPool
    from liteinfer_amd.cache.kv_cache import KVCache

    g = torch.Generator(device=DEV).manual_seed(9)
    pool = BlockPool(256, 16, 2, 8, 128, torch.bfloat16, DEV, cache_quant="fp8", k_scale=0.5, v_scale=0.25)
    cache = KVCache(pool)
    ids, prompts = ["a", "b", "c"], [37, 300, 129]
    cache.reserve(ids, prompts)
    payload = cache.make_packed_payload(ids, [0, 0, 0], prompts)
    t = sum(prompts)
    q = torch.randn(1, 32, t, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, 8, t, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, 8, t, 128, generator=g, device=DEV).to(torch.bfloat16)
    kv = payload.update(k, v, 1)
    assert kv.key_pool.dtype == FP8 and kv.k_scale == 0.5 and kv.v_scale == 0.25
    out = paged_attention(q, kv, 128 ** -0.5, 4)
    ref = eager_attention(q.float(), kv._replace(), 128 ** -0.5, 4)
    assert_within(out, to_numpy(ref).astype(np.float64), 2e-2, 2e-3)
    # A decode step over the same contexts, one new token each.
    totals = [p + 1 for p in prompts]
    cache.reserve(ids, totals)
    dec = cache.make_decode_payload(cache.newest_slots_for(ids, prompts), cache.slot_table_for(ids, totals),
                                    torch.tensor(totals, dtype=torch.int32, device=DEV))
    qd = torch.randn(3, 32, 1, 128, generator=g, device=DEV).to(torch.bfloat16)
    kd = torch.randn(3, 8, 1, 128, generator=g, device=DEV).to(torch.bfloat16)
    vd = torch.randn(3, 8, 1, 128, generator=g, device=DEV).to(torch.bfloat16)
    kvd = dec.update(kd, vd, 1)
    outd = paged_attention(qd, kvd, 128 ** -0.5, 4)
    refd = eager_attention(qd.float(), kvd, 128 ** -0.5, 4)
    assert_within(outd, to_numpy(refd).astype(np.float64), 2e-2, 2e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("batch", "tokens"), [(1, 37), (5, 1)])
def test_fused_rope_write_into_fp8_pools_is_rope_then_quantising_scatter(dtype, batch, tokens):
    """li_rope_kv_write_fp8 stores exactly what the torch rotation followed by the quantising
    slot-write stores, and returns the same rotated q as the bf16 / fp16 fused kernel."""
    from liteinfer_amd.rope import apply_rotary_pos_emb, rope_kv_write

    g = torch.Generator(device=DEV).manual_seed(10)
    heads, kvh, d, num_slots = 32, 8, 128, 512
    q = torch.randn(batch, tokens, heads, d, generator=g, device=DEV).to(dtype).transpose(1, 2)
    k = (torch.randn(batch, tokens, kvh, d, generator=g, device=DEV) * 20).to(dtype).transpose(1, 2)
    v = (torch.randn(batch, tokens, kvh, d, generator=g, device=DEV) * 20).to(dtype).transpose(1, 2)
    ang = torch.rand(batch, tokens, d, generator=g, device=DEV) * 6.28
    cos, sin = ang.cos().to(dtype), ang.sin().to(dtype)
    slots = torch.randperm(num_slots, device=DEV)[: batch * tokens].view(1, -1)
    kp = torch.zeros(num_slots, kvh, d, dtype=FP8, device=DEV)
    vp = torch.zeros_like(kp)
    q_out = rope_kv_write(q, k, v, cos, sin, slots, kp, vp, k_scale=0.5, v_scale=4.0)
    want_q, k_rot = apply_rotary_pos_emb(q, k, cos, sin)
    kp2, vp2 = torch.zeros_like(kp), torch.zeros_like(vp)
    kv_scatter(kp2, vp2, slots, k_rot, v, k_scale=0.5, v_scale=4.0)
    assert torch.equal(kp.view(torch.uint8), kp2.view(torch.uint8))
    assert torch.equal(vp.view(torch.uint8), vp2.view(torch.uint8))
    kp3 = torch.zeros(num_slots, kvh, d, dtype=dtype, device=DEV)
    q16 = rope_kv_write(q, k, v, cos, sin, slots, kp3, torch.zeros_like(kp3))
    assert torch.equal(q_out, q16) and torch.equal(q_out, want_q)


def test_fused_rope_write_into_fp8_pools_counts_slots_outside_the_pool():
    from liteinfer_amd.rope import rope_kv_write

    g = torch.Generator(device=DEV).manual_seed(12)
    q = torch.randn(1, 8, 4, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, 2, 4, 128, generator=g, device=DEV).to(torch.bfloat16)
    ang = torch.rand(1, 4, 128, generator=g, device=DEV)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    kp = torch.zeros(16, 2, 128, dtype=FP8, device=DEV)
    vp = torch.zeros_like(kp)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    rope_kv_write(q, k, k, cos, sin, torch.tensor([[2, 16, -3, 5]], device=DEV), kp, vp, bad_slots=bad)
    assert int(bad.item()) == 2
    written = (kp.view(torch.uint8) != 0).any(dim=(1, 2)).nonzero().reshape(-1).tolist()
    assert written == [2, 5]


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
def test_quantising_slot_write_passes_nan_through(src_dtype):
    """A NaN in K or V is stored as the e4m3 NaN (as torch's cast stores it),
    not clamped to a finite value that would hide the upstream error."""
    g = torch.Generator(device=DEV).manual_seed(5)
    k = torch.randn(2, 8, 3, 128, generator=g, device=DEV).to(src_dtype)
    v = torch.randn(2, 8, 3, 128, generator=g, device=DEV).to(src_dtype)
    k[0, 1, 2, 5] = float("nan")
    k[1, 7, 0, 127] = -float("nan")
    v[1, 0, 1, 64] = float("nan")
    kp = torch.zeros(16, 8, 128, dtype=torch.uint8, device=DEV).view(FP8)
    vp = torch.zeros_like(kp)
    slots = torch.tensor([[3, 9, 0, 15, 4, 7]], device=DEV)
    kv_scatter(kp, vp, slots, k, v)
    want_k = np.zeros((16, 8, 128), dtype=np.uint8)
    want_v = np.zeros((16, 8, 128), dtype=np.uint8)
    kf, vf = to_numpy(k).astype(np.float32), to_numpy(v).astype(np.float32)
    for i, s in enumerate(slots[0].tolist()):
        b, t = divmod(i, 3)
        want_k[s] = fp8.quantize(kf[b, :, t, :], 1.0)
        want_v[s] = fp8.quantize(vf[b, :, t, :], 1.0)
    # A NaN's sign is not defined (the hardware's conversion may set it), so
    # a NaN position must hold one of the two e4m3 NaN codes; every other
    # code is bit-exact.
    for got, want in ((_codes(kp), want_k), (_codes(vp), want_v)):
        nan = (want & 0x7F) == 0x7F
        assert np.array_equal(got[~nan], want[~nan])
        assert np.all((got[nan] & 0x7F) == 0x7F)
    assert nan.sum() == 1 and ((want_k & 0x7F) == 0x7F).sum() == 2


@pytest.mark.parametrize(("num_seqs", "num_heads", "num_kv_heads", "max_q", "max_prefix"), [
    (64, 8, 2, 60, 300),     # the most sequences the direct schedule scans
    (32, 32, 8, 32, 1500),   # 256 units (one block each): every CU one
    (5, 32, 8, 100, 90),     # several blocks a sequence, the first partial
    (65, 8, 1, 30, 200),     # one sequence too many: the work list again
])
def test_fp8_small_pass_without_a_work_list(num_seqs, num_heads, num_kv_heads, max_q, max_prefix):
    """An fp8 pool's small pass with no one-query rows in the launch: the lockstep kernel's direct
    schedule (each work-group finds its unit from the query counts; no work-list launch)."""
    from liteinfer_amd.paged_kernels import paged_prefill

    rng = np.random.default_rng(num_seqs + 3)
    q = rng.integers(1, max_q + 1, size=num_seqs).tolist()
    ctx = [qq + int(p) for qq, p in zip(q, rng.integers(0, max_prefix + 1, size=num_seqs))]
    b, kp, vp, want = _fp8_packed(ctx, q, 0.5, 0.25, num_heads=num_heads, num_kv_heads=num_kv_heads,
                                  seed=num_seqs, num_slots=1 << 17)
    out = paged_prefill(b.query, kp, vp, b.slot_table, b.context_lens_t, b.query_start_loc, max(q), b.scaling,
                        b.groups, k_scale=0.5, v_scale=0.25, one_query_rows=False)
    assert_within(out, want, 2e-2, 2e-3)
