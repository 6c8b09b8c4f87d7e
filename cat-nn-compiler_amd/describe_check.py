"""Checks describe() against a rocprofv3 kernel trace of bench.py.

For every node of the forward programs bench.py runs (configs 2, 3 and 4
and the Mixtral decoder), describe() names the kernels the node launches,
their grid and workgroup sizes, and the resources read from the build's
code objects.  The trace records what the GPU actually dispatched; this
script matches each described launch to a dispatch of the same kernel and
shape and compares workgroup, LDS, VGPR, AGPR and SGPR counts.

usage: python3 describe_check.py gpurun_out/trace/bench_kernel_trace.csv
(the trace of `rocprofv3 --kernel-trace ... -- python3 bench.py ...`).
"""
import csv
import os
import re
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from catnn_amd import configs, describe  # noqa: E402
from catnn_amd.configs import MixtralShape  # noqa: E402


def base_name(symbol):
    """The kernel's own identifier inside a mangled catnn::k::(anon)::name<...>."""
    m = re.match(r"_ZN5catnn1k(?:12_GLOBAL__N_1)?(\d+)", symbol)
    n = int(m.group(1))
    return symbol[m.end():m.end() + n]


def graphs():
    yield "config2", configs.config2().graph
    yield "config3", configs.config3().graph
    yield "config4", configs.config4().graph
    shape = MixtralShape(vocab=32000, hidden=1024, inter=3584, layers=2, heads=16, kv_heads=4, experts=8,
                         top_k=2, sliding_window=4096)
    yield "mixtral", configs.mixtral(batch=4, seq=2048, shape=shape).graph


def fused_into(g, op):
    return next(f.ops[0] for f in g.fusions if op in f.ops[1:])


GEMM_LIKE = ("linear", "matmul", "attention", "gqa_attention", "swiglu")


def residual_folded_into(g, nid):
    """The installed program folds a ResidualAdd into the GEMM that produces
    one operand when that operand has no other consumer and the other one
    comes earlier (graph.cpp, build_program); None when it does not."""
    node = g.nodes[nid]
    if node.op.kind != "residual_add":
        return None
    preds = g.preds(nid)
    order = g.topo()
    if len(preds) != 2 or preds[0] == preds[1]:
        return None
    for a, b in (preds, preds[::-1]):
        src = g.nodes[a]
        # a Linear fused with its activation produces through the activation node
        prod = next((g.nodes[p] for f in g.fusions if src.name in f.ops[1:]
                     for p in g.nodes if g.nodes[p].name == f.ops[0]), src)
        if prod.op.kind in GEMM_LIKE and len(g.succs(a)) == 1 and order.index(b) < order.index(a):
            return prod.name
    return None


def input_types(g, nid, dims):
    return [dims[e.src] for e in g.edges if e.dst == nid]


def main():
    trace = list(csv.DictReader(open(sys.argv[1])))
    seen = {}
    for r in trace:
        key = (r["Kernel_Name"], int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
        seen.setdefault(key, r)
    print("node                 kernel                      grid(items)   wg  static LDS(trace/desc) "
          "VGPR(trace/desc) AGPR SGPR(trace/desc) result")
    bad = 0
    for name, g in graphs():
        dims = {}
        for nid in g.topo():
            node = g.nodes[nid]
            if nid in g.inputs:
                dims[nid] = node.output_ty
                continue
            ins = input_types(g, nid, dims)
            dims[nid] = node.output_ty
            if any(node.name in f.ops[1:] for f in g.fusions):
                print(f"{name + ':' + node.name:20s} (fused into the GEMM epilogue of {fused_into(g, node.name)})")
                continue
            folded = residual_folded_into(g, nid)
            if folded is not None:
                print(f"{name + ':' + node.name:20s} (folded into the output GEMM of {folded})")
                continue
            r = describe(node, ins)
            for k in r.launches:
                bn = base_name(k.kernel)
                items = k.grid[0] * k.block[0]
                t = seen.get((bn, items, k.block[0]))
                if t is None:
                    print(f"{name + ':' + node.name:20s} {bn:27s} {items:11d} {k.block[0]:5d}   no dispatch of this "
                          f"shape in the trace   MISMATCH")
                    bad += 1
                    continue
                lds_t = int(t["LDS_Block_Size"])
                v_t, s_t = int(t["VGPR_Count"]), int(t["SGPR_Count"])
                # the dispatch record gives the static LDS in 512-byte granules and the unified
                # VGPR allocation as granules of 8 registers times 4; SGPRs are shown, not compared
                ok = lds_t == -(-k.static_lds_bytes // 512) * 512 and v_t == -(-k.vgprs // 8) * 4
                bad += not ok
                print(f"{name + ':' + node.name:20s} {bn:27s} {items:11d} {k.block[0]:5d} "
                      f"{lds_t:8d}/{k.static_lds_bytes:<8d} {v_t:4d}/{k.vgprs:<4d} {k.agprs:4d} "
                      f"{s_t:4d}/{k.sgprs:<4d} {'ok' if ok else 'MISMATCH'}")
    print(f"{bad} mismatches")
    sys.exit(1 if bad else 0)


if __name__ == "__main__":
    main()
