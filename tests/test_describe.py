"""describe() for the HIP backend (the counterpart of kernel::resource::
describe, crates/catnn-compile/src/kernel/resource.rs:155-186): the
kernels a node launches with the geometry the launchers choose, and each
kernel's resources read from this build's gfx950 code objects.  Host-only."""
import numpy as np
import pytest

from catnn_amd import (CatError, IrNode, OpenOp, Tensor, TensorType, configs, describe, kernel_table)


def _z(shape):
    return Tensor(TensorType.f32(shape), np.zeros(int(np.prod(shape)), np.float32))


def test_kernel_table_reads_the_code_objects():
    rows = kernel_table()
    assert len(rows) > 50
    names = [r.kernel for r in rows]
    assert len(set(names)) == len(names)
    for r in rows:
        assert r.code_bytes > 0 and r.kernarg_bytes > 0 and r.sgprs > 0, r.kernel
        assert r.block[0] in (256, 512, 1024), r.kernel
    # the fp32 MFMA GEMM keeps its accumulators in registers, no scratch; the
    # register-staged form declares its LDS, the direct-to-LDS form takes it at launch
    g = next(r for r in rows if "gemm_plain_kernelILi128ELi128ELi16ELb0ELb0E" in r.kernel)
    assert g.scratch_bytes_per_lane == 0 and g.vgprs >= 64 and g.static_lds_bytes > 0
    g = next(r for r in rows if "gemm_dma_kernelILi4ELb0ELb0E" in r.kernel)
    assert g.scratch_bytes_per_lane == 0 and g.vgprs >= 64 and g.static_lds_bytes == 0
    # the bf16 GEMM keeps its accumulators in AGPRs, counted inside the unified VGPR total
    b = next(r for r in rows if "gemm_bf16_kernelINS1_4DCfg" in r.kernel)
    assert 0 < b.agprs < b.vgprs


def test_linear_is_one_gemm_launch():
    # config 2's fc1: 8192 × 4096 → 16384 on 128 × 128 tiles
    node = IrNode(1, "fc1", OpenOp.linear(4096, 16384, True), TensorType.f32([8192, 16384]),
                  {"w": _z([4096, 16384]), "b": _z([16384])})
    r = describe(node, [TensorType.f32([8192, 4096])])
    assert len(r.launches) == 1
    k = r.launches[0]
    assert "gemm_dma_kernelILi4ELb0ELb0E" in k.kernel
    assert k.grid == (64 * 128, 1, 1) and k.block == (256, 1, 1)
    assert k.dynamic_lds_bytes == 4 * 16384
    assert r.code_bytes == k.code_bytes and not r.code_estimated
    assert r.registers_per_thread == k.vgprs  # unified VGPR + AGPR count
    assert r.scratch_bytes() == 4 * 16384 + r.registers_per_thread * 4 * 256
    # K not a multiple of 4: the register-staged element-load variant
    odd = IrNode(1, "fc", OpenOp.linear(7, 5, False), TensorType.f32([3, 5]), {"w": _z([7, 5])})
    assert "gemm_plain_kernelILi128ELi128ELi16ELb0ELb0E" in describe(odd, [TensorType.f32([3, 7])]).launches[0].kernel


def test_attention_block_and_moe_layer():
    w = configs.config3(batch=8, seq=1024, d=1024, heads=16, ffn=4096)
    attn = next(n for n in w.graph.nodes.values() if n.op.kind == "attention")
    r = describe(attn, [TensorType.f32([8, 1024, 1024])])
    kinds = [k.kernel for k in r.launches]
    assert len(kinds) == 3 and "attn_mfma_kernel" in kinds[1]
    assert r.launches[0].grid[0] == 64 * 24 and r.launches[1].grid[0] == 8 * 16 * 8
    assert r.temp_bytes == 8192 * 4 * 1024 * 4  # packed q|k|v and ctx
    m = configs.config4(batch=8, seq=2048, d=1024, n_experts=8, top_k=2, inter=3584)
    moe = m.graph.nodes[1]
    r = describe(moe, [TensorType.f32([8, 2048, 1024])])
    names = [k.kernel for k in r.launches]
    assert "route_dma_kernelILi2E" in names[0] and "combine4_kernel" in names[-1]
    dual = next(k for k in r.launches if "gemm_dma_kernelILi4ELb1ELb1E" in k.kernel)
    assert dual.grid[0] == (32768 // 128 + 8) * (3584 // 64)
    assert r.launches[0].dynamic_lds_bytes == 4 * (4 * 8 * 260 + 8 * (1024 + 4) + 32 * 8)
    assert r.code_bytes == sum({k.kernel: k.code_bytes for k in r.launches}.values())


def _every_kernel_path():
    """Nodes and input types that between them reach every pattern describe() names."""
    f = TensorType.f32
    ty = f([2, 8, 16])
    yield IrNode(1, "relu", OpenOp.relu(), ty), [ty]
    yield IrNode(1, "sm", OpenOp.softmax(-1), ty), [ty]
    yield IrNode(1, "sm_odd", OpenOp.softmax(-1), f([2, 8, 15])), [f([2, 8, 15])]
    yield IrNode(1, "add", OpenOp.add(), ty), [ty, ty]
    yield IrNode(1, "add_b", OpenOp.add(), ty), [ty, f([16])]
    yield IrNode(1, "mul", OpenOp.mul(), ty), [ty, ty]
    yield IrNode(1, "ln", OpenOp.layer_norm(1), ty, {"gamma": _z([16]), "beta": _z([16])}), [ty]
    yield IrNode(1, "ln_odd", OpenOp.layer_norm(1), f([4, 15]), {"gamma": _z([15]), "beta": _z([15])}), [f([4, 15])]
    yield (IrNode(1, "at", OpenOp.attention(4, 16, 4), ty, {p: _z([16, 16]) for p in ("wq", "wk", "wv", "wo")}),
           [ty])
    yield IrNode(1, "rms", OpenOp.rms_norm(10), f([3, 33]), {"w": _z([33])}), [f([3, 33])]
    yield IrNode(1, "rms4", OpenOp.rms_norm(10), f([3, 4096]), {"w": _z([4096])}), [f([3, 4096])]
    yield IrNode(1, "emb", OpenOp.embedding(50, 16), f([2, 4, 16]), {"w": _z([50, 16])}), [f([2, 4])]
    yield IrNode(1, "emb_odd", OpenOp.embedding(50, 6), f([2, 4, 6]), {"w": _z([50, 6])}), [f([2, 4])]
    yield IrNode(1, "emb1024", OpenOp.embedding(50, 1024), f([3, 1024]), {"w": _z([50, 1024])}), [f([3])]
    for hd in (6, 8, 64):  # RoPE one pair a thread (hd/2 odd), two pairs a thread
        d = 4 * hd
        yield (IrNode(1, f"gqa{hd}", OpenOp.gqa_attention(4, 2, hd, d, 8, 10000), f([2, 9, d]),
                      {"wq": _z([d, d]), "wk": _z([d, 2 * hd]), "wv": _z([d, 2 * hd]), "wo": _z([d, d])}),
               [f([2, 9, d])])
    for inter in (30, 32):  # register-staged dual tile, direct-to-LDS dual tile
        yield (IrNode(1, f"swiglu{inter}", OpenOp.swiglu(16, inter), ty,
                      {"w1": _z([16, inter]), "w3": _z([16, inter]), "w2": _z([inter, 16])}), [ty])
    yield IrNode(1, "lm", OpenOp.lm_head(16, 50), f([2, 8, 50]), {"w": _z([50, 16])}), [ty]
    yield IrNode(1, "mix", OpenOp.mix(), ty), [ty, ty]
    moe = {"gate": _z([10, 4])}
    for e in range(4):
        moe.update({f"e{e}.w1": _z([10, 12]), f"e{e}.w3": _z([10, 12]), f"e{e}.w2": _z([12, 10])})
    yield IrNode(1, "moe_odd", OpenOp.moe(4, 2, 10, 12), f([5, 10]), moe), [f([5, 10])]
    for E, H in ((4, 64), (16, 128), (8, 100)):  # staged router (64 and 16 tokens a block), streaming one
        moe = {"gate": _z([H, E])}
        for e in range(E):
            moe.update({f"e{e}.w1": _z([H, 8]), f"e{e}.w3": _z([H, 8]), f"e{e}.w2": _z([8, H])})
        yield IrNode(1, f"moe{E}", OpenOp.moe(E, 2, H, 8), f([40, H]), moe), [f([40, H])]


def test_every_kernel_named_resolves_once():
    seen = set()
    for node, ins in _every_kernel_path():
        r = describe(node, ins)
        assert r.launches, node.name
        for k in r.launches:
            assert k.code_bytes > 0 and k.grid[0] >= 1
            seen.add(k.kernel)
    assert any("route_kernel" in k for k in seen) and any("combine_kernel" in k for k in seen)
    assert any("route_vec_kernel" in k for k in seen)
    assert any("route_dma_kernelILi4E" in k for k in seen) and any("route_dma_kernelILi1E" in k for k in seen)
    assert any("attn_generic_kernel" in k for k in seen) and any("attn_mfma_kernel" in k for k in seen)
    assert any("rms_norm_any_kernel" in k for k in seen) and any("embedding_kernelILb0E" in k for k in seen)
    assert any("embedding_pair_kernel" in k for k in seen)
    assert any("rope_apply_kernel" in k for k in seen) and any("rope_apply2_kernel" in k for k in seen)
    assert any("gemm_grouped_kernel" in k for k in seen) and any("gemm_dma_kernelILi4ELb1ELb0E" in k for k in seen)
    # copies launch no kernel
    ty = TensorType.f32([2, 3])
    r = describe(IrNode(1, "t", OpenOp.transpose(0, 1), ty), [ty])
    assert r.launches == [] and r.code_bytes == 0


def test_describe_errors():
    ty = TensorType.f32([2, 8])
    with pytest.raises(CatError) as e:
        describe(IrNode(1, "mla", OpenOp("mla", (2, 4, 4, 4, 4, 4, 10000)), ty), [ty])
    assert e.value.kind == "Unsupported"
    with pytest.raises(CatError) as e:
        describe(IrNode(1, "fc", OpenOp.linear(9, 4, False), TensorType.f32([2, 4]), {"w": _z([9, 4])}), [ty])
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(CatError) as e:
        describe(IrNode(1, "ln", OpenOp.layer_norm(1), ty, {"beta": _z([8])}), [ty])
    assert e.value.kind == "UnknownPort"
