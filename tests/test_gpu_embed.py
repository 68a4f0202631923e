"""Gather-only embedding decode on the GPU (vqk_embed_gather) against the
oracle, bit-exact: VQEmbedding (vq_dense.py:444-513) over unpacked and
block-packed tables, VQPLEEmbedding (vq_switch.py:5426-5495) over uint16
and byte-stream rows, every output type, int32 / int64 ids, ids outside the
table, and the tied-head as_linear within the output tolerance."""
import numpy as np
import pytest

from oracle import vq_oracle as vo
from test_oracle import _stream_pack
from vq_cases import assert_close, make_module, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _bits(t):
    t = t.cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def _expect(w16, out_dtype):
    """fp16 oracle rows -> the bit patterns of out_dtype."""
    if out_dtype == torch.float16:
        return w16.view(np.uint16)
    if out_dtype == torch.bfloat16:
        return vo.f16_to_bf16(w16)
    return w16.astype(np.float32).view(np.uint32)


@pytest.mark.parametrize("D,K,packed,IN", [(2, 256, False, 4096), (4, 4096, True, 2048),
                                           (8, 16384, True, 1024), (8, 65536, False, 640),
                                           (4, 16, True, 80)])
@pytest.mark.parametrize("out_dtype", ["float16", "bfloat16", "float32"])
def test_vq_embedding_rows_bit_exact(D, K, packed, IN, out_dtype):
    from vqlab_amd.vq_dense import VQEmbedding
    print(f"VQEmbedding D={D} K={K} packed={packed} IN={IN} out={out_dtype}", flush=True)
    od = getattr(torch, out_dtype)
    rng = np.random.default_rng(D * 1000 + K % 997 + IN)
    G = 16 if IN == 80 else 64
    m = make_module(rng, 1, 300, IN, D, K, G=G, packed=packed)
    codes, cb, sc = to_device(m)
    emb = VQEmbedding(codes[0], cb, sc[0], group_size=G, pack_bits=m["pack_bits"],
                      in_features=IN if packed else None, out_dtype=od)
    assert emb.num_embeddings == 300 and emb.dims == IN
    ids = rng.integers(0, 300, (3, 5))
    for idt in (torch.int64, torch.int32):
        got = emb(torch.from_numpy(ids).to(idt).cuda())
        assert got.shape == (3, 5, IN) and got.dtype == od
        ref = vo.embed_rows(ids, m["codes"][0], m["codebook"], m["scales"][0], G)
        assert np.array_equal(_bits(got), _expect(ref, od))


def test_vq_embedding_ids_outside_table_give_zero_rows():
    from vqlab_amd.vq_dense import VQEmbedding
    rng = np.random.default_rng(5)
    m = make_module(rng, 1, 40, 256, 4, 256, packed=False)
    codes, cb, sc = to_device(m)
    emb = VQEmbedding(codes[0], cb, sc[0], out_dtype=torch.float16)
    ids = np.array([3, -1, 40, 39, 1 << 40])
    got = emb(torch.from_numpy(ids).cuda())
    ref = vo.embed_rows(np.array([3, 39]), m["codes"][0], m["codebook"], m["scales"][0], 64)
    g = _bits(got)
    assert np.array_equal(g[[0, 3]], ref.view(np.uint16))
    assert not g[[1, 2, 4]].any()


def test_vq_embedding_empty_ids_and_sharded_codebook():
    from vqlab_amd.vq_dense import VQEmbedding
    rng = np.random.default_rng(6)
    m = make_module(rng, 1, 16, 128, 4, 256, packed=False)
    codes, cb, sc = to_device(m)
    emb = VQEmbedding(codes[0], cb, sc[0])
    assert emb(torch.zeros((0,), dtype=torch.int64, device="cuda")).shape == (0, 128)
    emb.codebook = cb[:128]
    with pytest.raises(RuntimeError):
        emb(torch.zeros((2,), dtype=torch.int64, device="cuda"))


def test_vq_embedding_as_linear():
    from vqlab_amd.vq_dense import VQEmbedding
    rng = np.random.default_rng(7)
    m = make_module(rng, 1, 512, 1024, 8, 4096, packed=True)
    codes, cb, sc = to_device(m)
    emb = VQEmbedding(codes[0], cb, sc[0], pack_bits=m["pack_bits"], in_features=1024)
    x = rng.standard_normal((6, 1024)).astype(np.float32)
    y = emb.as_linear(torch.from_numpy(x).cuda())
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], 64)
    assert_close(y.cpu().numpy(), vo.decode_matmul(x, w), what="as_linear")


def _ple_table(rng, rows, nsub, d, K, G):
    codes = rng.integers(0, K, (rows, nsub)).astype(np.uint32)
    cb = (rng.standard_normal((K, d)) * 0.05).astype(np.float16)
    sc = rng.uniform(0.5, 1.5, (rows, nsub * d // G)).astype(np.float16)
    return codes, cb, sc


@pytest.mark.parametrize("K,d,packed", [(2048, 4, True), (4096, 4, True), (256, 4, True),
                                        (65536, 8, True), (8192, 2, False), (2048, 4, False)])
def test_vq_ple_embedding_bit_exact(K, d, packed):
    from vqlab_amd.vq_switch import VQPLEEmbedding
    print(f"VQPLEEmbedding K={K} d={d} packed={packed}", flush=True)
    rng = np.random.default_rng(K + d)
    nsub, rows = 40, 500
    G = 32 if (nsub * d) % 32 == 0 else 16
    codes, cb, sc = _ple_table(rng, rows, nsub, d, K, G)
    bits = max(1, (K - 1).bit_length())
    if packed:
        stored = torch.from_numpy(_stream_pack(codes, bits)).cuda()
        assert stored.shape[-1] == nsub * bits // 8
    else:
        stored = torch.from_numpy(codes.astype(np.uint16).view(np.int16)).cuda()
    ple = VQPLEEmbedding(stored, torch.from_numpy(cb).cuda(), torch.from_numpy(sc).cuda(),
                         group_size=G, packed_nsub=nsub if packed else 0)
    ids = rng.integers(0, rows, (2, 7))
    got = ple(torch.from_numpy(ids).cuda())
    assert got.dtype == torch.bfloat16 and got.shape == (2, 7, nsub * d)
    ref = vo.embed_rows(ids, codes, cb, sc, G)
    assert np.array_equal(_bits(got), vo.f16_to_bf16(ref))
