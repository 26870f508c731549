"""The W4A16 planner (t0_w4a16_plan, the kernel and split t0_w4a16_gemm
would launch) on the CPU, without a runtime (256 CUs assumed): the decode
kernel for M <= 64 with its row blocks and column tiles, split-K only where
the column blocks leave CUs idle and always dividing the quant groups, the
prefill tiles for M > 64, the generic kernel for the rest, and the refusals."""
import ctypes as C

import pytest

from t0_gpu._ffi import W4A16DescC, lib


def plan(m, n, k, gs=128, split_k=0, zeros=0, lda=0, scales_f32=0):
    d = W4A16DescC(a=0, qweight=0, scales=0, zeros=zeros, c=0, m=m, n=n, k=k, lda=lda, ldc=0, group_size=gs,
                   zero_const=8, scales_f32=scales_f32, out_f32=0, split_k=split_k)
    name, sk = C.create_string_buffer(96), C.c_uint32()
    rc = lib().t0_w4a16_plan(None, C.byref(d), name, 96, C.byref(sk))
    if rc:
        raise ValueError(lib().t0_last_error().decode())
    return name.value.decode(), sk.value


@pytest.mark.parametrize("m,mb", [(1, 1), (16, 1), (17, 2), (32, 2), (33, 4), (64, 4)])
def test_decode_row_blocks(m, mb):
    name, _ = plan(m, 11008, 4096)
    assert name == f"t0k_w4a16_decode_t3_mb{mb}"


@pytest.mark.parametrize("n,tiles", [(1024, 1), (4096, 1), (5120, 2), (8192, 2), (11008, 3), (12288, 3),
                                     (14336, 4), (28672, 4)])
def test_decode_column_tiles(n, tiles):
    """One workgroup per CU over an even share of N's 4-column units, the
    fewest 16-column tiles that hold a share (at most 4: wider N takes more
    workgroups of 64 columns)."""
    units = n // 4
    wgs = min(256, (n + 15) // 16)
    want = -(-4 * -(-units // wgs) // 16)
    if want > 4:
        want = 4
    assert tiles == want
    name, _ = plan(16, n, 4096)
    assert name == f"t0k_w4a16_decode_t{tiles}_mb1"


@pytest.mark.parametrize("n,k", [(512, 4096), (1024, 1024), (1024, 4096), (2048, 11008), (4096, 4096),
                                 (11008, 4096), (256, 14336), (128, 512)])
def test_decode_split_k_fills_idle_cus_and_divides_the_groups(n, k):
    _, sk = plan(16, n, k)
    groups = k // 128
    wgs = min(256, (n + 15) // 16)
    assert sk >= 1 and sk & (sk - 1) == 0 and groups % sk == 0
    assert wgs * sk <= 256
    assert groups // sk >= 4                       # a pipeline stage or more per partition
    # doubling would break one of the three
    assert wgs * sk * 2 > 256 or groups % (2 * sk) or groups // (2 * sk) < 4


def test_explicit_split_k():
    assert plan(16, 1024, 4096, split_k=4)[1] == 4
    with pytest.raises(ValueError, match="divide"):
        plan(16, 1024, 4096, split_k=3)


@pytest.mark.parametrize("m,name", [(65, "t0k_w4a16_prefill_128x128_w2x2_s2"),
                                    (1023, "t0k_w4a16_prefill_128x128_w2x2_s2"),
                                    (1024, "t0k_w4a16_prefill_128x256_w1x8_s3"),
                                    (4096, "t0k_w4a16_prefill_128x256_w1x8_s3")])
def test_prefill_tiles(m, name):
    assert plan(m, 14336, 4096) == (name, 1)


@pytest.mark.parametrize("kw", [dict(gs=64), dict(lda=4100), dict(n=1004)])
def test_generic_kernel_for_the_rest(kw):
    args = dict(m=16, n=1024, k=4096)
    args.update(kw)
    assert plan(**args)[0] == "t0k_w4a16_generic"


@pytest.mark.parametrize("kw,msg", [(dict(k=4100), "K"), (dict(gs=12), "gs"), (dict(k=4160, gs=128), "K"),
                                    (dict(m=0), "empty"), (dict(n=1004, zeros=256), "N")])
def test_refusals(kw, msg):
    args = dict(m=16, n=1024, k=4096)
    args.update(kw)
    with pytest.raises(ValueError, match=msg):
        plan(**args)
