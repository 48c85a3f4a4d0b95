"""CPU tests of the C-ABI boundary: the library loads, exports every symbol include/lrm_hip.h declares, and its
host-side contract checks follow the reference's Lrm.Gpu.Core rules and vectors (docs/contracts/kernel-abi.md
"Vectors", heap-and-tensor-table.md "Vectors"). No compute call needs a GPU here.
"""
import ctypes
import hashlib
import json
import os
import re

import numpy as np
import pytest

from conftest import GOLDEN, ROOT
from oracle import cpuref
from rosylnalive_amd import _native
from rosylnalive_amd.gpu_core import (Arena, ArgBlock, Catalog, DType, GpuContractException, HeapLayout, HeapPlanner,
                                      TensorFlags, TensorTable, grid_physical, prepare)
from rosylnalive_amd.qwen import QWEN3_INV_FREQ_HD128, inv_freq_bits, rope_table, synthetic_normal_f32

VEC = json.load(open(os.path.join(GOLDEN, "reference_vectors.json")))
GiB = 1 << 30


def declared_functions():
    src = open(_native.HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(lrm_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_native.LIB_PATH)
    names = declared_functions()
    assert len(names) > 50
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes prototypes cover exactly the header
    assert set(names) == set(_native.PROTOTYPES), set(names) ^ set(_native.PROTOTYPES)


def test_abi_version_and_catalog_order():
    L = _native.lib()
    assert L.lrm_abi_version() == 1
    names = [k.name for k in Catalog.all()]
    # Kernels.all at contracts-v1 (kernel-abi.md "The catalog at contracts-v1"), then the appended fast-path kernels
    assert names[:14] == ["scale_f32", "table_echo", "args_echo", "groups_echo", "bf16_unpack", "embed_gather_bf16",
                          "rmsnorm_rows", "rope_apply", "silu_mul", "add", "copy_rows", "argmax_rows", "matmul_bf16w",
                          "attention_gqa_causal"]
    threads = [k.threads for k in Catalog.all()[:14]]
    assert threads == [(256, 1, 1), (16, 1, 1), (32, 1, 1), (1, 1, 1), (256, 1, 1), (256, 1, 1), (256, 1, 1),
                       (64, 1, 1), (256, 1, 1), (256, 1, 1), (256, 1, 1), (256, 1, 1), (16, 16, 1), (64, 1, 1)]
    linear = [k.name for k in Catalog.all()[:14] if k.linear]
    assert linear == ["scale_f32", "table_echo", "args_echo", "groups_echo", "bf16_unpack", "rmsnorm_rows", "rope_apply",
                      "silu_mul", "add", "copy_rows", "argmax_rows"]
    assert len(Catalog.find("args_echo").fields) == 31
    assert len(names) == len(set(names))


def test_grid_folding_edge_cases():
    assert grid_physical(True, 65535, 1, 1) == (65535, 1, 1)
    assert grid_physical(True, 65536, 1, 1) == (32768, 2, 1)
    assert grid_physical(True, 70000, 1, 1) == (35000, 2, 1)
    with pytest.raises(GpuContractException):
        grid_physical(False, 70000, 1, 1)
    with pytest.raises(GpuContractException):
        grid_physical(True, 0, 1, 1)
    rng = np.random.default_rng(0)
    for x in rng.integers(65536, 65535 * 65535, 50):
        px, py, _ = grid_physical(True, int(x), 1, 1)
        assert px * py >= x and px * py - x < py and px <= 65535


def _table(specs, pages=None):
    """A table over a layout of 1 GiB pages: specs = [(name, dtype, dims, flags)], one tensor per page."""
    pages = pages or [(Arena.ACTIVATIONS, GiB)] * len(specs)
    layout = HeapLayout.of_pages(pages)
    t = TensorTable(layout)
    toks = [t.add(n, i + 1, 0, d, dims, f) for i, (n, d, dims, f) in enumerate(specs)]
    return t.seal(), toks


def test_argblock_vectors_A1_to_A4():
    # A1 scale_f32 {x = t5; y = t6; n = 1000; a = 0.5}
    specs = [(f"t{i}", DType.F32, [1024], 0) for i in range(1, 7)]
    sealed, _ = _table(specs)
    words, grid, phys = prepare(sealed, Catalog.find("scale_f32").id, ArgBlock.encode("scale_f32", x=5, y=6, n=1000, a=0.5))
    assert ["%08x" % w for w in words[:5]] == ["00000004", "00000005", "00000006", "000003e8", "3f000000"]
    assert words[5:] == [0] * 27 and phys == (4, 1, 1)
    # A2 matmul_bf16w {x = t1; w = t2; y = t3; m = 37; n = 151936; k = 1024}
    sealed, _ = _table([("x", DType.F32, [37, 1024], 0), ("w", DType.BF16, [151936, 1024], 0),
                        ("y", DType.F32, [37, 151936], 0)])
    words, grid, phys = prepare(sealed, 12, ArgBlock.encode("matmul_bf16w", x=1, w=2, y=3, m=37, n=151936, k=1024))
    assert ["%08x" % w for w in words[:7]] == ["00000946", "00000001", "00000002", "00000003", "00000025", "00025180",
                                               "00000400"]
    assert phys == (2374, 1, 1)
    # A3 add {a = t1; b = t2; y = t3; n = 8192 * 3072}: 98,304 groups folded to (49152, 2, 1)
    n = 8192 * 3072
    sealed, _ = _table([(f"t{i}", DType.F32, [n], 0) for i in range(1, 4)])
    words, grid, phys = prepare(sealed, 9, ArgBlock.encode("add", a=1, b=2, y=3, n=n))
    assert ["%08x" % w for w in words[:5]] == ["0000c000", "00000001", "00000002", "00000003", "01800000"]
    assert grid == (98304, 1, 1) and phys == (49152, 2, 1)
    # A4 attention_gqa_causal {rows = 7; q_row0 = 0; past = 0; q_heads = 16; kv_heads = 8; head_dim = 128}
    sealed, _ = _table([("q", DType.F32, [7, 2048], 0), ("k", DType.F32, [7, 1024], 0), ("v", DType.F32, [7, 1024], 0),
                        ("y", DType.F32, [7, 2048], 0)])
    scale = float(np.float32(1 / np.sqrt(128)))
    words, grid, phys = prepare(sealed, 13, ArgBlock.encode("attention_gqa_causal", q=1, k=2, v=3, y=4, rows=7, q_row0=0,
                                                            past=0, q_heads=16, kv_heads=8, head_dim=128, scale=scale))
    assert ["%08x" % w for w in words[:12]] == ["00000007", "00000001", "00000002", "00000003", "00000004", "00000007",
                                                "00000000", "00000000", "00000010", "00000008", "00000080", "3db504f3"]
    assert phys == (7, 16, 1)


def test_dispatch_rules_raise_contract_errors():
    sealed, _ = _table([("x", DType.F32, [1024], 0), ("w", DType.BF16, [1024], TensorFlags.READ_ONLY),
                        ("y", DType.F32, [1024], 0), ("ro", DType.F32, [1024], TensorFlags.READ_ONLY)])
    ok = ArgBlock.encode("scale_f32", x=1, y=3, n=1000, a=2.0)
    prepare(sealed, 0, ok)
    bad = ArgBlock(ok.words)
    bad.words[0] = 5  # word 0 is written by Dispatch
    with pytest.raises(GpuContractException, match="word 0"):
        prepare(sealed, 0, bad)
    bad = ArgBlock(ok.words)
    bad.words[7] = 1  # past the last field
    with pytest.raises(GpuContractException, match="past the last field"):
        prepare(sealed, 0, bad)
    with pytest.raises(GpuContractException, match="null token"):
        prepare(sealed, 0, ArgBlock.encode("scale_f32", x=0, y=3, n=4, a=1.0))
    with pytest.raises(GpuContractException, match="not in the table"):
        prepare(sealed, 0, ArgBlock.encode("scale_f32", x=9, y=3, n=4, a=1.0))
    with pytest.raises(GpuContractException, match="does not accept"):
        prepare(sealed, 0, ArgBlock.encode("scale_f32", x=2, y=3, n=4, a=1.0))  # bf16 into an f32 field
    with pytest.raises(GpuContractException, match="read only"):
        prepare(sealed, 0, ArgBlock.encode("scale_f32", x=1, y=4, n=4, a=1.0))
    with pytest.raises(GpuContractException, match="elements"):
        prepare(sealed, 0, ArgBlock.encode("scale_f32", x=1, y=3, n=2000, a=1.0))  # minimum element counts
    with pytest.raises(GpuContractException, match="empty"):
        prepare(sealed, 0, ArgBlock.encode("scale_f32", x=1, y=3, n=0, a=1.0))
    # aliasing: scale_f32's y may alias x (the same bytes); matmul_bf16w's y may not alias its input
    prepare(sealed, 0, ArgBlock.encode("scale_f32", x=1, y=1, n=1000, a=2.0))
    with pytest.raises(GpuContractException, match="overlap"):
        prepare(sealed, 12, ArgBlock.encode("matmul_bf16w", x=1, w=2, y=1, m=1, n=1, k=4))


def test_attention_combine_splits_bound():
    """The partials hold max_pos / 64 splits per head: an even-split count past that is a contract error."""
    sealed, _ = _table([("part", DType.F32, [16 * 2 * 130], 0), ("y", DType.F16, [2048], 0),
                        ("state", DType.U32, [4], TensorFlags.READ_ONLY)])
    kid = 35  # attention_combine_f16
    for splits in (0, 1, 2):
        prepare(sealed, kid, ArgBlock.encode("attention_combine_f16", partials=1, y=2, state=3, q_heads=16,
                                             max_pos=128, batch=1, chunks=0, splits=splits))
    with pytest.raises(GpuContractException, match="splits"):
        prepare(sealed, kid, ArgBlock.encode("attention_combine_f16", partials=1, y=2, state=3, q_heads=16,
                                             max_pos=128, batch=1, chunks=0, splits=3))


def test_a_shift_bound():
    """The SwiGLU output's producers and consumers take its shift (a_shift, in binades) up to 24; past that the
    dispatch is a contract error."""
    sealed, _ = _table([("a", DType.F16, [16 * 1024], 0), ("w", DType.F16, [1024 * 1024], TensorFlags.READ_ONLY),
                        ("x", DType.F32, [2 * 16 * 1024], 0), ("y", DType.F16, [16 * 512], 0)])
    cases = [("gemm_residual", dict(a=1, w=2, x=3, m=16, n=1024, k=1024)),
             ("gemm_swiglu", dict(a=1, w=2, y=4, m=16, inter=512, k=1024)),
             ("gemm_skinny_residual", dict(a=1, w=2, x=3, m=16, n=1024, k=1024)),
             ("gemm_skinny_swiglu", dict(a=1, w=2, y=4, m=16, inter=512, k=1024)),
             ("gemm_residual_split", dict(a=1, w=2, partials=3, m=16, n=1024, k=1024, splits=2))]
    for name, f in cases:
        kid = Catalog.find(name).id
        for s in (0, 8, 24):
            prepare(sealed, kid, ArgBlock.encode(name, a_shift=s, **f))
        with pytest.raises(GpuContractException, match="a_shift must be at most 24"):
            prepare(sealed, kid, ArgBlock.encode(name, a_shift=25, **f))


def test_tensor_row_vectors_T1_T2():
    out = (ctypes.c_uint32 * 16)()
    dims = (ctypes.c_uint32 * 2)(151936, 1024)
    _native.check(_native.lib().lrm_tensor_row(1, 256, DType.BF16, dims, 2, TensorFlags.READ_ONLY,
                                               b"model.embed_tokens.weight", out))
    assert " ".join("%08x" % int.from_bytes(int(w).to_bytes(4, "little"), "big") for w in out) == (
        "01000000 00010000 02000000 02000000 80510200 00040000 01000000 01000000 "
        "00040000 01000000 00000000 00000000 00004609 03000000 fcd443ac 00000000")
    dims = (ctypes.c_uint32 * 3)(7, 16, 128)
    _native.check(_native.lib().lrm_tensor_row(4, 4096, DType.F32, dims, 3, TensorFlags.VIEW, b"L0.attn.q_rope", out))
    assert " ".join("%08x" % int.from_bytes(int(w).to_bytes(4, "little"), "big") for w in out) == (
        "04000000 00100000 01000000 03000000 07000000 10000000 80000000 01000000 "
        "00080000 80000000 01000000 00000000 00380000 05000000 d4fd8611 00000000")
    assert _native.lib().lrm_debug_id(b"") == 0


def test_planner_and_table_rules():
    p = HeapPlanner(1 << 20)
    a = p.allocate(Arena.WEIGHTS, 1000)
    b = p.allocate(Arena.WEIGHTS, 1000)
    c = p.allocate(Arena.WEIGHTS, (1 << 20) - 100)  # does not fit the rest of page 0: a new page
    d = p.allocate(Arena.ACTIVATIONS, 64)
    assert (a[1], a[2]) == (0, 0) and (b[1], b[2]) == (0, 1024) and (c[1], c[2]) == (1, 0) and (d[1], d[2]) == (0, 0)
    layout = p.build()
    assert [(pg.arena, pg.bytes) for pg in layout.pages] == [(1, 64 << 10), (1, 1 << 20), (4, 64 << 10)]
    with pytest.raises(GpuContractException):
        p.allocate(Arena.WEIGHTS, 10)  # after build
    with pytest.raises(GpuContractException, match="reserved"):
        HeapPlanner().allocate(Arena.MASTER, 10)
    t = TensorTable(layout)
    t1 = t.add_placed("w", a, DType.BF16, [500], TensorFlags.READ_ONLY)
    t2 = t.add_view("w.view", t1, [100], 10)
    assert (t1, t2) == (1, 2)
    with pytest.raises(GpuContractException, match="already"):
        t.add_placed("w", b, DType.BF16, [500])
    with pytest.raises(GpuContractException, match="inside"):
        t.add_view("bad.view", t1, [600], 0)
    with pytest.raises(GpuContractException, match="page"):
        t.add("too.big", 1, 0, DType.F32, [1 << 20])  # past the 64 KiB page
    sealed = t.seal()
    assert len(sealed.image) == 1 << 20 and sealed.row(0) == [0] * 16
    r = sealed.row(t2)
    assert r[0] == 1 and r[1] == 20 and r[13] == TensorFlags.CONTIGUOUS | TensorFlags.VIEW | TensorFlags.READ_ONLY
    with pytest.raises(GpuContractException):
        t.seal()
    with pytest.raises(GpuContractException, match="contract order"):
        TensorTable(HeapLayout.of_pages([(Arena.ACTIVATIONS, 64 << 10), (Arena.WEIGHTS, 64 << 10)]))


def test_product_rope_table_is_t_spec():
    """The product's own T_spec builder (not the oracle) against the reference digests and the oracle's table."""
    cos, sin = rope_table(128, 8192)
    assert hashlib.sha256(cos.tobytes() + sin.tobytes()).hexdigest() == VEC["qwen_table_digest_8192"]
    inv = inv_freq_bits(32)
    assert ["%08x" % w for w in inv] == ["%08x" % int(h, 16) for h in VEC["qwen_inv_freq_hd128"][::4]]
    c32, s32 = rope_table(32, 512)
    assert hashlib.sha256(c32.tobytes() + s32.tobytes()).hexdigest() == VEC["tiny_table_digest_512"]
    oc, os_ = cpuref.rope_table(inv_freq_bits(16), 300)
    pc, ps = rope_table(16, 300)
    assert oc.tobytes() == pc.tobytes() and os_.tobytes() == ps.tobytes()
    assert hashlib.sha256(np.array(QWEN3_INV_FREQ_HD128, np.uint32).tobytes()).hexdigest() == VEC["qwen_inv_freq_sha256"]


def test_synthetic_inputs_are_deterministic_normals():
    a = synthetic_normal_f32(7, "probe", (400000,))
    b = synthetic_normal_f32(7, "probe", (400000,))
    c = synthetic_normal_f32(8, "probe", (400000,))
    assert a.tobytes() == b.tobytes() and a.tobytes() != c.tobytes()
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    # a prefix of a longer draw is the shorter draw: element values depend only on (seed, stream, index)
    assert synthetic_normal_f32(7, "probe", (1001,)).tobytes() == a[:1001].tobytes()


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 exits with status 2 and says so, before touching a device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2, (r.returncode, r.stdout, r.stderr)
    assert "one GPU" in (r.stdout + r.stderr)
    assert r.stdout.strip() == ""  # no JSON line
