"""sai_copy_rows on the GPU: rows between [B, H, S, D] and [B, S, H*D] with a
sequence offset (kv_concat / kv_copy_block and reshape_to_bhsd /
reshape_from_bhsd, onnx-rt/src/ops/microsoft.rs:660-792), checked bit for
bit against numpy transposes. Untouched destination rows keep their fill."""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


def bhsd(x, layout, b, h, s, d):
    """The [B, H, S, D] view of rows stored in `layout`."""
    return x.reshape(b, h, s, d) if layout == S.ROPE_BHSD else \
        x.reshape(b, s, h, d).transpose(0, 2, 1, 3)


@pytest.mark.parametrize("src_layout", [S.ROPE_BHSD, S.ROPE_BSHD])
@pytest.mark.parametrize("dst_layout", [S.ROPE_BHSD, S.ROPE_BSHD])
@pytest.mark.parametrize("dtype,d,offset", [("f32", 128, 0), ("bf16", 64, 0), ("f32", 6, 0),
                                            ("f32", 128, 1), ("bf16", 128, 1)])
def test_copy_rows_bit_exact(rt, src_layout, dst_layout, dtype, d, offset):
    import torch
    log(f"copy_rows {src_layout}->{dst_layout} {dtype} d={d} ptr offset {offset}")
    rng = np.random.default_rng(d + offset)
    b, h, s, dst_seq, off = 3, 4, 7, 12, 5
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    x = torch.from_numpy(rng.standard_normal(b * h * s * d).astype(np.float32)).to(tdt)
    src_buf = torch.zeros(x.numel() + offset, dtype=tdt)
    src_buf[offset:] = x
    src = src_buf.cuda()[offset:]
    dst_buf = torch.full((b * h * dst_seq * d + offset,), 9.0, dtype=tdt, device="cuda")
    dst = dst_buf[offset:]
    rt.copy_rows(src, src_layout, dst, dst_layout, b, h, s, d, dst_seq, off)
    torch.cuda.synchronize()
    got = bhsd(dst.float().cpu().numpy(), dst_layout, b, h, dst_seq, d)
    want = bhsd(x.float().numpy(), src_layout, b, h, s, d)
    assert np.array_equal(got[:, :, off:off + s], want)
    assert np.all(got[:, :, :off] == 9.0) and np.all(got[:, :, off + s:] == 9.0)


def test_copy_rows_concat_and_errors(rt):
    """past [B,H,P,D] ++ new [B,S,H*D] -> present [B,H,P+S,D] in two calls."""
    import torch
    b, h, p, s, d = 2, 8, 33, 3, 128
    past = torch.randn(b, h, p, d, device="cuda")
    new = torch.randn(b, s, h * d, device="cuda")
    present = torch.empty(b, h, p + s, d, device="cuda")
    rt.copy_rows(past, S.ROPE_BHSD, present, S.ROPE_BHSD, b, h, p, d, p + s, 0)
    rt.copy_rows(new, S.ROPE_BSHD, present, S.ROPE_BHSD, b, h, s, d, p + s, p)
    torch.cuda.synchronize()
    want = torch.cat([past, new.reshape(b, s, h, d).transpose(1, 2)], dim=2)
    assert torch.equal(present, want)
    with pytest.raises(S.SaiError) as e:
        rt.copy_rows(new, S.ROPE_BSHD, present, S.ROPE_BHSD, b, h, s, d, p + s, p + 1)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(S.SaiError) as e:
        rt.copy_rows(new, 3, present, S.ROPE_BHSD, b, h, s, d, p + s, 0)
    assert e.value.kind == "InvalidAttribute"
