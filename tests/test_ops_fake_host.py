"""Host tests of the `register_fake` implementations (what torch.compile traces):
under FakeTensorMode each registered op must report the output shape and dtype
the reference op returns for the same arguments.  Expected shapes follow the
reference registrations: (1, M, inner) for the joint-attention ops with M the
token count (op_fused_attention.py:95-108, single_stream/.../op_fused_attention.py:84-86),
(M, Hq*D) for the backbone attention (op_fused_llm_attention.py:30-45),
per-group (M, N_half) for ds::grouped_swiglu (op_grouped_swiglu.py:40-49).
The GPU test test_gpu_ops.py::test_register_fake_matches_real_op checks the
same fakes against the real ops."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import rldx_amd.ops  # noqa: F401

BF16 = torch.bfloat16


def e(*shape, dtype=BF16):
    return torch.empty(*shape, dtype=dtype)


@pytest.mark.parametrize("lead", [(82,), (1, 82)])
def test_ss_fused_attention_2way_fake_counts_every_leading_dim(lead):
    with FakeTensorMode():
        o = torch.ops.ss.fused_attention_2way(e(*lead, 4608), e(64), e(64), e(18, 32, dtype=torch.float32),
                                              e(18, 32, dtype=torch.float32), 18)
    assert tuple(o.shape) == (1, 82, 1536) and o.dtype == BF16


def test_joint_attention_fakes():
    with FakeTensorMode():
        f32 = lambda n: e(n, 32, dtype=torch.float32)  # noqa: E731
        o2 = torch.ops.ds.fused_attention_2way(e(1, 18, 4608), e(1, 64, 4608), e(64), e(64), e(64), e(64), f32(18),
                                               f32(18), 18, 64)
        o3 = torch.ops.ds.fused_attention_3way(e(18, 4608), e(64, 4608), e(16, 4608), *(e(64) for _ in range(6)),
                                               f32(18), f32(18), f32(16), f32(16), 18, 64, 16)
        s3 = torch.ops.ss.fused_attention_3way(e(82, 4608), e(16, 4608), *(e(64) for _ in range(4)), f32(18), f32(18),
                                               f32(16), f32(16), 82, 18, 16)
        w = torch.ops.ds.fused_attention_2way(e(64, 4608), e(512, 4608), e(128), e(128), e(128), e(128),
                                              e(64, 64, dtype=torch.float32), e(64, 64, dtype=torch.float32), 64, 512,
                                              num_heads=12, head_dim=128)
    assert tuple(o2.shape) == (1, 82, 1536)
    assert tuple(o3.shape) == (1, 98, 1536)
    assert tuple(s3.shape) == (1, 98, 1536)
    assert tuple(w.shape) == (1, 576, 1536)


def test_backbone_and_mlp_fakes():
    with FakeTensorMode():
        b = torch.ops.rldx_backbone.fused_attention(e(169, (32 + 16) * 128), e(128), e(128), e(128), e(128),
                                                    e(169, 128), e(169, 128))
        g = torch.ops.ds.grouped_swiglu(e(18, 8192), e(8192), e(64, 21844), e(21844), 18, 64, 4096, 10922)
        m = torch.ops.ss.fused_mlp_swiglu(e(82, 1536), e(2 * 6144, 1536), e(2 * 6144))
        s = torch.ops.rldx_amd.swiglu(e(1, 82, 2 * 6144))
        v = torch.ops.rldx_backbone.vision_attention(e(392, 3 * 16 * 72), e(392, 72, dtype=torch.float32),
                                                     e(392, 72, dtype=torch.float32), e(3, dtype=torch.int32),
                                                     72 ** -0.5, 16, 72)
        mm = torch.ops.mem.fused_attention(e(64, 3 * 16 * 256), e(64, 256), e(64, 256), 16, 256, 16)
    assert tuple(b.shape) == (169, 4096)
    assert tuple(g[0].shape) == (18, 4096) and tuple(g[1].shape) == (64, 10922)
    assert tuple(m.shape) == (82, 6144)
    assert tuple(s.shape) == (1, 82, 6144)
    assert tuple(v.shape) == (392, 1152)
    assert tuple(mm.shape) == (64, 4096)


def test_epilogue_fakes():
    with FakeTensorMode():
        sa, vl = torch.ops.ds.grouped_res_ln(e(18, 1536), e(1536), e(18, 1536), e(64, 4096), e(4096), e(64, 4096),
                                             18, 64, 1536, 4096)
        nv, lv = torch.ops.ds.vl_epilogue_ln(e(64, 4096), e(4096), e(4096), e(64, 4096), 64, 4096)
        nh, ln = torch.ops.ss.fused_epilogue_ln(e(1, 82, 1536), e(1, 82, 1536))
        a2 = torch.ops.rldx_backbone.fused_epilogue_add2_rmsnorm(e(169, 4096), e(169, 4096), e(4096))
        a3 = torch.ops.rldx_backbone.fused_epilogue_add3_rmsnorm(e(169, 4096), e(169, 4096), e(169, 4096), e(4096))
        m2 = torch.ops.mem.fused_epilogue_add2_rmsnorm(e(1, 64, 2048), e(1, 64, 2048), e(2048))
    assert tuple(sa.shape) == (1, 18, 1536) and tuple(vl.shape) == (1, 64, 4096)
    assert tuple(nv.shape) == (1, 64, 4096) and tuple(lv.shape) == (1, 64, 4096)
    assert tuple(nh.shape) == (1, 82, 1536) and tuple(ln.shape) == (1, 82, 1536)
    assert all(tuple(t.shape) == (169, 4096) for t in (*a2, *a3))
    assert all(tuple(t.shape) == (1, 64, 2048) for t in m2)
