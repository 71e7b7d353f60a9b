"""The C11 host engine of libpyc_amd.so against the reference's own engine.

The reference engine (oracle/_ref/libpyc_ref.so, built from the reference
sources) is the checker: identical call sequences go through both libraries
and every observable result is compared - IR verification codes and
serialisation, pass reports and transformed modules, allocator plans,
controller transitions, registry selections and scores, CPU-executor outputs
(bit for bit), decision logs and run stats. The reference's own C tests are
ported alongside (their numbers are cited inline)."""
import ctypes as C

import numpy as np
import pytest

from pyc_amd import abi
from tests import engine_util as eu

needs_ref = pytest.mark.skipif(not eu.ref_available(), reason="oracle/_ref not built here")
LIBS = ["mine", "ref"]


def lib(name):
    return eu.mine() if name == "mine" else eu.ref()


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for k in ("PYC_CUDA_SIMULATE_AVAILABLE", "PYC_CUDA_DISABLE", "PYC_CUDA_FORCE_FALLBACK", "PYC_CUDA_FORCE_ERROR",
              "PYC_NUM_THREADS", "PYC_HIP_STRICT", "PYC_AUTOTUNE_DB_PATH", "PYC_COMPILE_DELAY_MS"):
        monkeypatch.delenv(k, raising=False)


# ---------------------------------------------------------------- IR


def _modules(seed):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(20):
        n_in = int(r.integers(1, 4))
        ops = [eu.op(abi.OP_INPUT, f"in{i}", tuple(int(x) for x in r.integers(1, 9, int(r.integers(1, 3)))))
               for i in range(n_in)]
        for j in range(int(r.integers(1, 6))):
            kind = int(r.choice([abi.OP_ADD, abi.OP_RELU, abi.OP_GELU, abi.OP_CONST, abi.OP_LAYERNORM]))
            src = int(r.integers(0, len(ops)))
            ins = (src, int(r.integers(0, len(ops)))) if kind == abi.OP_ADD else (src,)
            ops.append(eu.op(kind, "" if r.random() < 0.3 else f"op{j}", (), ins))
        ops.append(eu.op(abi.OP_OUTPUT, "out", (), (len(ops) - 1,)))
        out.append(ops)
    return out


@needs_ref
def test_ir_verify_codes_match_reference():
    cases = [
        [],  # empty -> 2
        [eu.op(abi.OP_INPUT, "a", (0, 3))],  # bad dim -> 4
        [eu.op(abi.OP_INPUT, "a", (2,)), eu.op(abi.OP_RELU, "r", (), (1,))],  # forward ref -> 5
        [eu.op(abi.OP_INPUT, "a", (2,)), eu.op(abi.OP_RELU, "r", (), (-1,))],  # negative -> 5
        [eu.op(abi.OP_INPUT, "a", (2, 2)), eu.op(abi.OP_OUTPUT, "o", (), (0,))],  # ok
    ]
    codes = {}
    for name in LIBS:
        L = lib(name)
        codes[name] = []
        for ops in cases:
            m = eu.module(ops)
            d = abi.IrDiagnostic()
            rc = L.pyc_ir_verify(C.byref(m), C.byref(d))
            codes[name].append((rc, d.code, d.message))
    assert codes["mine"] == codes["ref"]
    assert [c[1] for c in codes["mine"]] == [2, 4, 5, 5, 0]  # reference tests/compiler_next/test_ir.c


@needs_ref
def test_ir_serialize_matches_reference():
    for ops in _modules(1):
        m = eu.module(ops)
        assert eu.serialize(eu.mine(), m) == eu.serialize(eu.ref(), m)


# ---------------------------------------------------------------- passes


GOLDEN = ("0:input:lhs:dtype=1:shape=2x3:inputs=\n1:input:rhs:dtype=1:shape=3x4:inputs=\n"
          "2:matmul:fused_op_2_op_3:dtype=1:shape=2x4:inputs=0,1\n3:output:op_4:dtype=1:shape=2x4:inputs=2\n")


def _golden_module():
    return eu.module([eu.op(abi.OP_INPUT, "lhs", (2, 3)), eu.op(abi.OP_INPUT, "rhs", (3, 4)),
                      eu.op(abi.OP_MATMUL, "", (), (0, 1)), eu.op(abi.OP_RELU, "", (), (2,)),
                      eu.op(abi.OP_OUTPUT, "", (), (3,))])


def _run_passes(L, m, fusion=1):
    cfg = eu.PassConfig(1, 1, 1, fusion, 1, 1, 1)
    rep = eu.PassReport()
    rc = L.pyc_pass_pipeline_run(C.byref(cfg), C.byref(m), C.byref(rep))
    return rc, rep


def test_pass_golden_fusion_output():
    """reference tests/compiler_next/test_pass_golden.c + golden/simple_pipeline_after.txt"""
    m = _golden_module()
    rc, rep = _run_passes(eu.mine(), m)
    assert rc == 0 and rep.fused_patterns == 1
    assert eu.serialize(eu.mine(), m) == GOLDEN


@needs_ref
@pytest.mark.parametrize("fusion", [0, 1])
def test_pass_reports_match_reference(fusion):
    mats = [[eu.op(abi.OP_INPUT, "x", (4, 8)), eu.op(abi.OP_INPUT, "w", (8, 5)), eu.op(abi.OP_INPUT, "b", (5,)),
             eu.op(abi.OP_MATMUL, "mm", (), (0, 1)), eu.op(abi.OP_ADD, "add", (), (3, 2)),
             eu.op(abi.OP_GELU, "", (), (4,)), eu.op(abi.OP_OUTPUT, "o", (), (5,))]]
    for ops in _modules(2) + mats:
        m1, m2 = eu.module(ops), eu.module(ops)
        rc1, r1 = _run_passes(eu.mine(), m1, fusion)
        rc2, r2 = _run_passes(eu.ref(), m2, fusion)
        assert rc1 == rc2
        assert bytes(r1) == bytes(r2)
        assert eu.serialize(eu.mine(), m1) == eu.serialize(eu.ref(), m2)


# ---------------------------------------------------------------- allocator


def _plan(L, reqs, mode, budget):
    plan = eu.AllocPlan()
    L.pyc_alloc_plan_init(C.byref(plan))
    for r in reqs:
        L.pyc_alloc_plan_add_request(C.byref(plan), eu.AllocRequest(*r))
    L.pyc_alloc_plan_build_with_mode(C.byref(plan), mode, budget)
    st = eu.AllocStats()
    L.pyc_alloc_plan_stats(C.byref(plan), C.byref(st))
    return list(plan.offsets[:plan.request_count]), bytes(st)


@needs_ref
def test_allocator_plans_match_reference():
    r = np.random.default_rng(3)
    for _ in range(60):
        reqs = []
        for i in range(int(r.integers(1, 24))):
            s = int(r.integers(0, 10))
            reqs.append((i, int(r.integers(1, 5000)), int(r.choice([1, 16, 64, 256])), s, s + int(r.integers(0, 4))))
        budget = int(r.choice([0, 1000, 8000, 30000]))
        for mode in (abi.MODE_BALANCED, abi.MODE_MEMORY_FIRST, abi.MODE_UTILIZATION_FIRST):
            assert _plan(eu.mine(), reqs, mode, budget) == _plan(eu.ref(), reqs, mode, budget)


def test_allocator_reuse_reference_case():
    """reference tests/compiler_next/test_runtime_allocator.c: disjoint lifetimes share memory."""
    offs, st = _plan(eu.mine(), [(0, 1024, 64, 0, 1), (1, 1024, 64, 2, 3), (2, 512, 64, 1, 2)], 0, 0)
    stats = eu.AllocStats.from_buffer_copy(st)
    assert offs[1] == offs[0] and stats.reused_allocations == 1 and stats.peak_bytes == 1536


# ---------------------------------------------------------------- controller


def _control_trace(L, seq, rails_tweak):
    rails = abi.RuntimeRails()
    L.pyc_runtime_rails_default(C.byref(rails))
    for k, v in rails_tweak.items():
        setattr(rails, k, v)
    ctl = eu.Controller()
    L.pyc_runtime_controller_init(C.byref(ctl), abi.MODE_BALANCED)
    out = []
    for m in seq:
        met = eu.WindowMetrics(*m)
        mode, why = C.c_int(), C.c_int()
        L.pyc_runtime_controller_observe(C.byref(ctl), C.byref(rails), C.byref(met), C.byref(mode), C.byref(why))
        out.append((mode.value, why.value, bytes(ctl)))
    return out


@needs_ref
def test_controller_matches_reference():
    r = np.random.default_rng(4)
    for trial in range(30):
        seq = []
        for _ in range(40):
            seq.append((10.0, float(r.choice([9.0, 10.5, 12.0])), 100.0, float(r.choice([80.0, 99.0, 120.0])),
                        float(r.choice([0.0, 0.1, 0.5])), int(r.choice([0, 0, 1])), int(r.choice([0, 0, 5])),
                        int(r.random() < 0.05)))
        tweak = {"dwell_steps": int(r.integers(1, 5)), "cooldown_steps": int(r.integers(0, 3)),
                 "enable_hard_rollback": int(trial % 2)}
        assert _control_trace(eu.mine(), seq, tweak) == _control_trace(eu.ref(), seq, tweak)


# ---------------------------------------------------------------- registry


def _desc(symbol, prio, occ, lds, reg, wl=0, hw=0, tc=0):
    d = abi.KernelDesc()
    d.op_key = b"matmul_fused"
    d.backend = abi.BACKEND_CPU
    d.symbol = symbol.encode()
    d.priority = prio
    d.estimated_occupancy = occ
    d.shared_mem_bytes = lds
    d.reg_pressure_class = reg
    d.preferred_workload_family = wl
    d.preferred_hardware_family = hw
    d.tensor_core_eligible = tc
    return d


def _registry_scenario(L):
    """reference tests/compiler_next/test_kernel_registry.c, step by step."""
    out, tr, bench = abi.KernelDesc(), abi.KernelSelectionTrace(), abi.KernelBenchmark()
    got = []
    L.pyc_kernel_registry_reset()
    L.pyc_kernel_register(C.byref(_desc("kernel_v1", 5, 0.5, 48 * 1024, 3)))
    L.pyc_kernel_register(C.byref(_desc("kernel_v2", 10, 0.9, 4 * 1024, 1)))
    L.pyc_kernel_select(b"matmul_fused", 0, C.byref(out))
    got.append(out.symbol)
    prom = C.create_string_buffer(128)
    got.append(L.pyc_kernel_promote_symbol(b"matmul_fused", 0, b"kernel_v1"))
    L.pyc_kernel_promoted_symbol(b"matmul_fused", 0, prom, 128)
    got.append(prom.value)
    got.append(L.pyc_kernel_promote_symbol(b"matmul_fused", 0, b"kernel_missing"))
    L.pyc_kernel_benchmark_update(b"matmul_fused", 0, 1.2)
    L.pyc_kernel_benchmark_update(b"matmul_fused", 0, 0.9)
    L.pyc_kernel_select_with_policy(b"matmul_fused", 0, abi.MODE_MEMORY_FIRST, 4.0, C.byref(out), C.byref(tr))
    got += [out.symbol, bytes(tr)]
    ctx = abi.CoselectContext(2.5, 2, 3, 1, 4096, 4096, 2048, 0, 0)
    L.pyc_kernel_register(C.byref(_desc("kernel_co_high_pressure", 20, 0.98, 96 * 1024, 4)))
    L.pyc_kernel_register(C.byref(_desc("kernel_co_memory_friendly", 14, 0.72, 2 * 1024, 1)))
    L.pyc_kernel_select_with_policy(b"matmul_fused", 0, abi.MODE_BALANCED, 2.5, C.byref(out), None)
    got.append(out.symbol)
    L.pyc_kernel_coselect_with_context(b"matmul_fused", 0, abi.MODE_MEMORY_FIRST, C.byref(ctx), C.byref(out),
                                       C.byref(tr))
    got += [out.symbol, bytes(tr)]
    L.pyc_kernel_register(C.byref(_desc("kernel_square_hopper", 14, 0.7, 8192, 1, abi.WL_LARGE_SQUARE, abi.HW_HOPPER)))
    L.pyc_kernel_register(C.byref(_desc("kernel_tall_generic", 14, 0.7, 8192, 1, abi.WL_TALL_SKINNY, abi.HW_GENERIC)))
    ctx.workload_family, ctx.hardware_family = abi.WL_LARGE_SQUARE, abi.HW_HOPPER
    L.pyc_kernel_coselect_with_context(b"matmul_fused", 0, abi.MODE_BALANCED, C.byref(ctx), C.byref(out), C.byref(tr))
    got.append(out.symbol)
    ctx.workload_family, ctx.hardware_family = abi.WL_TALL_SKINNY, abi.HW_GENERIC
    L.pyc_kernel_coselect_with_context(b"matmul_fused", 0, abi.MODE_BALANCED, C.byref(ctx), C.byref(out), C.byref(tr))
    got.append(out.symbol)
    L.pyc_kernel_benchmark_read(b"matmul_fused", 0, C.byref(bench))
    got.append(bytes(bench))
    descs = (abi.KernelDesc * 16)()
    n = L.pyc_kernel_collect(b"matmul_fused", 0, descs, 16)
    got.append([descs[i].symbol for i in range(n)])
    return got


def test_registry_reference_scenario():
    got = _registry_scenario(eu.mine())
    assert got[0] == b"kernel_v2" and got[1] == 0 and got[2] == b"kernel_v1" and got[3] == -1
    assert got[4] == b"kernel_v2"
    assert got[6] == b"kernel_co_high_pressure" and got[7] == b"kernel_co_memory_friendly"
    assert got[9] == b"kernel_square_hopper" and got[10] == b"kernel_tall_generic"
    assert got[12] == sorted(got[12])
    eu.mine().pyc_kernel_registry_reset()


@needs_ref
def test_registry_matches_reference():
    assert _registry_scenario(eu.mine()) == _registry_scenario(eu.ref())
    r = np.random.default_rng(5)
    for L in (eu.mine(), eu.ref()):
        L.pyc_kernel_registry_reset()
    descs = [_desc(f"k{i:02d}", int(r.integers(0, 20)), float(r.random()), int(r.integers(0, 128)) * 1024,
                   int(r.integers(0, 5)), int(r.integers(0, 6)), int(r.integers(0, 4)), int(r.integers(0, 2)))
             for i in range(24)]
    for d in descs:
        for L in (eu.mine(), eu.ref()):
            L.pyc_kernel_register(C.byref(d))
    for _ in range(50):
        ctx = abi.CoselectContext(float(r.choice([0.0, 0.3, 2.0])), int(r.integers(0, 3)), int(r.integers(0, 3)),
                                  int(r.integers(0, 5)), int(r.integers(0, 10000)), int(r.integers(0, 10000)),
                                  int(r.choice([0, 5000])), int(r.integers(0, 6)), int(r.integers(0, 4)))
        mode = int(r.integers(0, 3))
        res = []
        for L in (eu.mine(), eu.ref()):
            out, tr = abi.KernelDesc(), abi.KernelSelectionTrace()
            L.pyc_kernel_coselect_with_context(b"matmul_fused", 0, mode, C.byref(ctx), C.byref(out), C.byref(tr))
            res.append((out.symbol, bytes(tr)))
        assert res[0] == res[1]
    for L in (eu.mine(), eu.ref()):
        L.pyc_kernel_registry_reset()


# ---------------------------------------------------------------- engine, CPU backend


def _mlp_ops(m, k, n, add_shape=None, relu=True):
    ops = [eu.op(abi.OP_INPUT, "lhs", (m, k)), eu.op(abi.OP_INPUT, "rhs", (k, n))]
    if add_shape:
        ops.append(eu.op(abi.OP_INPUT, "addend", add_shape))
    ops.append(eu.op(abi.OP_MATMUL, "matmul0", (), (0, 1)))
    last = len(ops) - 1
    if add_shape:
        ops.append(eu.op(abi.OP_ADD, "add0", (), (last, 2)))
        last = len(ops) - 1
    if relu:
        ops.append(eu.op(abi.OP_RELU, "relu0", (), (last,)))
        last = len(ops) - 1
    ops.append(eu.op(abi.OP_OUTPUT, "out0", (m, n), (last,)))
    return ops


def test_cpu_execution_kats():
    """reference tests/compiler_next/test_cpu_execution.c:56-59 and :135-138."""
    L = eu.mine()
    mdl = eu.Model(L, _mlp_ops(2, 3, 2, relu=False))
    st, (out,), stats = mdl.run([np.array([[1, 2, 3], [4, 5, 6]], np.float32),
                                 np.array([[1, 2], [3, 4], [5, 6]], np.float32)], [(2, 2)])
    mdl.close()
    assert st == 0 and out.tolist() == [[22, 28], [49, 64]]
    ops = [eu.op(abi.OP_INPUT, "a", (4,)), eu.op(abi.OP_INPUT, "b", (4,)), eu.op(abi.OP_ADD, "add", (), (0, 1)),
           eu.op(abi.OP_RELU, "relu", (), (2,)), eu.op(abi.OP_OUTPUT, "o", (4,), (3,))]
    mdl = eu.Model(L, ops)
    st, (out,), _ = mdl.run([np.array([-1, 2, -3, 4], np.float32), np.array([2, -5, 4, -1], np.float32)], [(4,)])
    mdl.close()
    assert st == 0 and out.tolist() == [1, 0, 1, 3]


@needs_ref
@pytest.mark.parametrize("threads", [None, "4"])
def test_cpu_engine_matches_reference_bitwise(monkeypatch, threads):
    if threads:
        monkeypatch.setenv("PYC_NUM_THREADS", threads)
    r = np.random.default_rng(6)
    for m, k, n in [(2, 3, 2), (16, 40, 24), (33, 70, 9)]:
        a = r.uniform(-1, 1, (m, k)).astype(np.float32)
        b = r.uniform(-1, 1, (k, n)).astype(np.float32)
        c = r.uniform(-1, 1, (m, n)).astype(np.float32)
        res = {}
        for name in LIBS:
            mdl = eu.Model(lib(name), _mlp_ops(m, k, n, add_shape=(m, n)))
            assert mdl.status == 0
            st1, (o1,), s1 = mdl.run([a, b, c], [(m, n)])
            st2, (o2,), s2 = mdl.run([a, b, c], [(m, n)])
            res[name] = (st1, st2, o1.copy(), o2.copy(), eu.log_fields(mdl.log()), s2)
            mdl.close()
        mine, ref = res["mine"], res["ref"]
        assert mine[0] == ref[0] == 0 and mine[1] == ref[1] == 0
        np.testing.assert_array_equal(mine[2], ref[2])
        np.testing.assert_array_equal(mine[3], ref[3])
        lm, lr = mine[4], ref[4]
        assert list(lm.keys()) == list(lr.keys())
        for key in ("mode", "kernel", "score", "util", "alloc_penalty", "workload", "hw", "cuda_fallback", "contract",
                    "contract_reason", "guard_miss", "fallback", "graph_breaks", "compilability", "fp"):
            assert lm[key] == lr[key], key
        sm, sr = mine[5], ref[5]
        for f in ("peak_bytes", "total_requested_bytes", "reused_allocations", "selected_kernel_score",
                  "model_fingerprint", "graph_break_count", "compilability_score", "selected_kernel_symbol",
                  "deterministic_contract_ok", "guard_miss_count", "fallback_count", "speculative_shape_bucket"):
            assert getattr(sm, f) == getattr(sr, f), f


@needs_ref
def test_guards_and_statuses_match_reference():
    a = np.ones((4, 8), np.float32)
    b = np.ones((8, 3), np.float32)
    for name in LIBS:
        L = lib(name)
        assert L.pyc_status_string(4) == b"RUNTIME_FAILED"
        mdl = eu.Model(L, _mlp_ops(4, 8, 3, relu=False))
        st, _, stats = mdl.run([a, np.ones((8, 4), np.float32)], [(4, 3)])  # wrong rhs shape
        assert st == abi.STATUS_RUNTIME_FAILED
        assert stats.guard_miss_count == 1 and stats.deterministic_contract_reason == b"input_shape_mismatch"
        st, _, stats = mdl.run([a, b], [(4, 3)])
        assert st == 0
        mdl.close()
        bad = eu.Model(L, [eu.op(abi.OP_INPUT, "a", (2,)), eu.op(abi.OP_RELU, "r", (), (3,))])
        assert bad.status == abi.STATUS_VERIFY_FAILED


@needs_ref
def test_speculative_and_phantom_match_reference():
    r = np.random.default_rng(7)
    a = r.uniform(-1, 1, (4, 8)).astype(np.float32)
    b = r.uniform(-1, 1, (8, 4)).astype(np.float32)
    fields = ("speculative_plan_count", "speculative_plan_hit", "speculative_plan_miss_count",
              "phantom_graph_enabled", "phantom_graph_match", "phantom_graph_match_count",
              "phantom_graph_mismatch_count", "phantom_graph_reshape_count", "phantom_graph_match_score",
              "phantom_graph_expected_signature", "phantom_graph_observed_signature", "speculative_shape_bucket")
    res = {}
    for name in LIBS:
        mdl = eu.Model(lib(name), _mlp_ops(4, 8, 4, relu=False), enable_speculative_plans=1,
                       enable_phantom_graph=1, phantom_horizon_steps=1)
        seq = []
        st, _, s = mdl.run([a, b], [(4, 4)])
        seq.append((st, tuple(getattr(s, f) for f in fields)))
        st, _, s = mdl.run([a, b], [(4, 4)])
        seq.append((st, tuple(getattr(s, f) for f in fields)))
        res[name] = seq
        mdl.close()
    assert res["mine"] == res["ref"]
    assert res["mine"][0][1][1] == 1  # plan hit on the compiled shape


@needs_ref
def test_compile_cache_matches_reference(monkeypatch):
    """reference tests/compiler_next/test_compile_cache.c: the second compile of the
    same module/options is a cache hit and much faster under PYC_COMPILE_DELAY_MS."""
    monkeypatch.setenv("PYC_COMPILE_DELAY_MS", "30")
    for name in LIBS:
        L = lib(name)
        ops = _mlp_ops(3, 5, 7)
        ops[0].name = f"uniq_{name}".encode()
        m1 = eu.Model(L, ops, cache_mode=abi_cache_in_memory())
        m2 = eu.Model(L, ops, cache_mode=abi_cache_in_memory())
        st1, _, s1 = m1.run([np.ones((3, 5), np.float32), np.ones((5, 7), np.float32)], [(3, 7)])
        st2, _, s2 = m2.run([np.ones((3, 5), np.float32), np.ones((5, 7), np.float32)], [(3, 7)])
        assert st1 == st2 == 0
        assert s1.compile_cache_hit == 0 and s2.compile_cache_hit == 1
        assert s1.compile_ms >= 25.0 and s2.compile_ms < s1.compile_ms
        m1.close()
        m2.close()


def abi_cache_in_memory():
    return 1  # PYC_COMPILE_CACHE_IN_MEMORY


def test_autotune_db_persists_and_reloads(tmp_path):
    L = eu.mine()
    db = str(tmp_path / "tune.db")
    mdl = eu.Model(L, _mlp_ops(4, 4, 4, relu=False), enable_autotune=1, autotune_db_path=db.encode())
    for _ in range(3):
        st, _, s = mdl.run([np.ones((4, 4), np.float32), np.ones((4, 4), np.float32)], [(4, 4)])
        assert st == 0
    assert s.autotune_saved == 1
    mdl.close()
    lines = open(db).read().strip().splitlines()
    assert lines and all(len(l.split("|")) == 4 and l.split("|")[0] == "matmul_fused" for l in lines)
    assert len({l.split("|")[2] for l in lines}) == len(lines)  # compacted: one row per symbol
    mdl = eu.Model(L, _mlp_ops(4, 4, 4, relu=False), enable_autotune=1, autotune_db_path=db.encode())
    st, _, s = mdl.run([np.ones((4, 4), np.float32), np.ones((4, 4), np.float32)], [(4, 4)])
    assert s.autotune_loaded == 1
    mdl.close()


# ---------------------------------------------------------------- GPU backend contract (no device here)


KAT_LHS = np.array([[1, -2], [3, 4]], np.float32)
KAT_RHS = np.array([[2, 1], [-1, 3]], np.float32)
KAT_BIAS = np.array([0.5, -1.5], np.float32)
KAT_OUT = [[4.5, 0.0], [2.5, 13.5]]


def _kat_model(L):
    return eu.Model(L, _mlp_ops(2, 2, 2, add_shape=(2,)), backend=abi.BACKEND_CUDA, fusion=1)


@needs_ref
def test_backend_simulated_contract_matches_reference(monkeypatch):
    """reference tests/compiler_next/test_cuda_backend.c with PYC_CUDA_SIMULATE_AVAILABLE
    (no device in this container): KAT, replay, fallback and forced error."""
    monkeypatch.setenv("PYC_CUDA_SIMULATE_AVAILABLE", "1")
    monkeypatch.setenv("PYC_CUDA_ASSUME_STATIC_RHS", "1")
    for name in LIBS:
        L = lib(name)
        mdl = _kat_model(L)
        for _ in range(2):
            st, (out,), s = mdl.run([KAT_LHS, KAT_RHS, KAT_BIAS], [(2, 2)])
            assert st == 0 and s.fallback_count == 0, name
            np.testing.assert_allclose(out, KAT_OUT, atol=1e-5)
            lf = eu.log_fields(mdl.log())
            assert lf["cuda_fallback"] == "0" and lf["cuda_reason"] == "cuda_native_simulated", name
        monkeypatch.setenv("PYC_CUDA_FORCE_FALLBACK", "1")
        st, (out,), s = mdl.run([KAT_LHS, KAT_RHS, KAT_BIAS], [(2, 2)])
        lf = eu.log_fields(mdl.log())
        assert st == 0 and s.fallback_count == 1 and lf["cuda_reason"] == "cuda_forced_fallback", name
        monkeypatch.setenv("PYC_CUDA_FORCE_ERROR", "1")
        st, _, s = mdl.run([KAT_LHS, KAT_RHS, KAT_BIAS], [(2, 2)])
        assert st == abi.STATUS_RUNTIME_FAILED, name
        assert eu.log_fields(mdl.log())["cuda_reason"] == "forced_error", name
        monkeypatch.delenv("PYC_CUDA_FORCE_ERROR")
        monkeypatch.delenv("PYC_CUDA_FORCE_FALLBACK")
        monkeypatch.setenv("PYC_CUDA_DISABLE", "1")
        monkeypatch.delenv("PYC_CUDA_SIMULATE_AVAILABLE")
        st, _, s = mdl.run([KAT_LHS, KAT_RHS, KAT_BIAS], [(2, 2)])
        lf = eu.log_fields(mdl.log())
        assert st == 0 and lf["cuda_fallback"] == "1" and lf["cuda_reason"] == "disabled_by_env", name
        monkeypatch.delenv("PYC_CUDA_DISABLE")
        monkeypatch.setenv("PYC_CUDA_SIMULATE_AVAILABLE", "1")
        mdl.close()


def test_backend_bf16_passthrough_simulated(monkeypatch):
    """reference tests/compiler_next/test_cuda_backend.c:252-312 (bit-exact bf16 passthrough)."""
    monkeypatch.setenv("PYC_CUDA_SIMULATE_AVAILABLE", "1")
    L = eu.mine()
    ops = [eu.op(abi.OP_INPUT, "input0", (4,), dtype=abi.DTYPE_BF16),
           eu.op(abi.OP_OUTPUT, "output0", (4,), (0,), dtype=abi.DTYPE_BF16)]
    mdl = eu.Model(L, ops, backend=abi.BACKEND_CUDA)
    data = np.array([0x3F80, 0x4000, 0x4040, 0x4080], np.uint16)
    st, (out,), s = mdl.run([data], [(4,)], in_dtypes=[abi.DTYPE_BF16], out_dtypes=[abi.DTYPE_BF16],
                            out_np_dtype=np.uint16)
    mdl.close()
    assert st == 0 and s.fallback_count == 0 and out.tolist() == data.tolist()


def test_strict_mode_turns_fallback_into_error(monkeypatch):
    monkeypatch.setenv("PYC_CUDA_DISABLE", "1")
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    mdl = _kat_model(eu.mine())
    st, _, s = mdl.run([KAT_LHS, KAT_RHS, KAT_BIAS], [(2, 2)])
    mdl.close()
    assert st == abi.STATUS_RUNTIME_FAILED and s.fallback_count == 1


def test_unsupported_kind_reason(monkeypatch):
    monkeypatch.setenv("PYC_CUDA_SIMULATE_AVAILABLE", "1")
    ops = [eu.op(abi.OP_INPUT, "x", (4,)), eu.op(abi.OP_REDUCE_SUM, "r", (), (0,)), eu.op(abi.OP_OUTPUT, "o", (1,), (1,))]
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)
    st, _, s = mdl.run([np.ones(4, np.float32)], [(1,)])
    lf = eu.log_fields(mdl.log())
    mdl.close()
    # REDUCE_SUM has no lowering anywhere: the CPU executor refuses it too
    assert st == abi.STATUS_RUNTIME_FAILED and lf["cuda_reason"] == "cpu_fallback_failed"
    assert s.graph_break_reduce_sum_count == 1


def test_graph_break_op_falls_back_to_cpu_executor(monkeypatch):
    """GELU is a graph break for the reference (pass_manager.c:313-373) and its
    executor refuses it; this engine's CPU executor runs it, so without a GPU
    the module completes as a CPU fallback."""
    import oracle
    monkeypatch.setenv("PYC_CUDA_DISABLE", "1")
    ops = [eu.op(abi.OP_INPUT, "x", (4,)), eu.op(abi.OP_GELU, "g", (), (0,)), eu.op(abi.OP_OUTPUT, "o", (4,), (1,))]
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)
    x = np.array([-2.0, -0.5, 0.0, 3.0], np.float32)
    st, (out,), s = mdl.run([x], [(4,)])
    lf = eu.log_fields(mdl.log())
    mdl.close()
    assert st == 0 and lf["cuda_fallback"] == "1" and lf["cuda_reason"] == "disabled_by_env"
    assert s.graph_break_gelu_count == 1
    assert np.allclose(out, oracle.gelu_f64(x.astype(np.float64)), rtol=1e-6, atol=1e-7)


def test_engine_wrapper_cpu_backend():
    """pyc_amd.engine (the Python side of the run path that bench.py's engine
    workload uses) on the CPU backend: matmul+bias+ReLU through
    pyc_compile_model/pyc_run_model equals the oracle's CPU executor result bit
    for bit, and run_stats_json carries the reference bench driver's fields."""
    import oracle
    from pyc_amd import abi, engine

    M, K, N = 16, 24, 8
    r = np.random.default_rng(3)
    x, w = r.uniform(-1, 1, (M, K)).astype(np.float32), r.uniform(-1, 1, (K, N)).astype(np.float32)
    b = r.uniform(-1, 1, N).astype(np.float32)
    ops = [engine.op(abi.OP_INPUT, "x", (M, K)), engine.op(abi.OP_INPUT, "w", (K, N)),
           engine.op(abi.OP_INPUT, "bias", (N,)), engine.op(abi.OP_MATMUL, "matmul0", (), (0, 1)),
           engine.op(abi.OP_ADD, "add0", (), (3, 2)), engine.op(abi.OP_RELU, "relu0", (), (4,)),
           engine.op(abi.OP_OUTPUT, "out0", (M, N), (5,))]
    model = engine.Model(ops, backend=abi.BACKEND_CPU)
    assert model.status == 0
    y = np.zeros((M, N), np.float32)
    stats, wall = [], []
    for _ in range(3):
        rc, st = model.run([engine.host_tensor(a, abi.DTYPE_F32) for a in (x, w, b)],
                           [engine.host_tensor(y, abi.DTYPE_F32)])
        assert rc == 0
        stats.append(st)
        wall.append(st.run_ms)
    ref = np.maximum(oracle.matmul_f32(x, w) + b[None, :], 0.0)
    assert np.array_equal(y, ref.astype(np.float32))
    j = engine.run_stats_json(stats, wall, model)
    model.close()
    for key in ("latency_ms", "peak_memory_bytes", "profile", "controller", "execution_path", "kernel_selection",
                "compile_options", "reliability", "phantom_graph", "precision_policy"):
        assert key in j, key
    assert set(j["latency_ms"]) == {"mean", "p50", "p95", "min", "max"}
    assert j["execution_path"].startswith("cpu"), j["execution_path"]


def test_hip_autotune_without_gpu():
    """pyc_hip_autotune_gemm times nothing without a GPU (returns 0) and rejects
    bad arguments; the engine's per-run autotune record stays in force then."""
    import pyc_amd
    L = pyc_amd.lib()
    f = L.pyc_hip_autotune_gemm
    f.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_size_t, C.POINTER(C.c_double), C.c_int]
    f.restype = C.c_int
    syms, ms = C.create_string_buffer(64 * 4), (C.c_double * 4)()
    assert f(abi.DTYPE_BF16, 0, 8, 8, 1, syms, 64, ms, 4) == -1
    assert f(abi.DTYPE_I32, 8, 8, 8, 1, syms, 64, ms, 4) == -1
    import torch
    if not torch.cuda.is_available():
        assert f(abi.DTYPE_BF16, 8, 8, 8, 1, syms, 64, ms, 4) == 0


def test_stable_repeat_fastpath_many_inputs(monkeypatch):
    """A module with more inputs than the reference's stable-repeat cap (8
    inputs; this engine takes the fast path up to 64): repeats with identical
    descriptors take the fast path, which must still read the inputs' current
    contents, and a changed descriptor (a new buffer, a wrong shape) must go
    through the full guard path again. The reference engine, which never
    takes the fast path at this size, gives the same statuses and outputs."""
    monkeypatch.setenv("PYC_CUDA_DISABLE", "1")  # the GPU backend's CPU fallback, with or without a device
    n = 12
    ops = [eu.op(abi.OP_INPUT, f"x{i}", (4,)) for i in range(n)]
    cur = 0
    for i in range(1, n):
        ops.append(eu.op(abi.OP_ADD, f"a{i}", (), (cur, i)))
        cur = len(ops) - 1
    ops.append(eu.op(abi.OP_OUTPUT, "o", (4,), (cur,)))
    results = {}
    for name in LIBS if eu.ref_available() else ["mine"]:
        L = lib(name)
        mdl = eu.Model(L, ops, backend=abi.BACKEND_CUDA)
        xs = [np.full(4, float(i + 1), np.float32) for i in range(n)]
        y = np.zeros(4, np.float32)

        def run(inputs):
            ins = (abi.Tensor * len(inputs))(*[eu.tensor(a, abi.DTYPE_F32) for a in inputs])
            outs = (abi.Tensor * 1)(eu.tensor(y, abi.DTYPE_F32))
            s = abi.RunStats()
            return L.pyc_run_model(mdl.h, ins, len(inputs), outs, 1, C.byref(s)), y.copy()

        seq = [run(xs) for _ in range(3)]
        xs[5][:] = 100.0  # same buffer, new contents
        seq.append(run(xs))
        xs[7] = np.full(4, -3.0, np.float32)  # a new buffer
        seq.append(run(xs))
        bad = list(xs)
        bad[3] = np.zeros(5, np.float32)  # wrong shape
        seq.append(run(bad))
        seq.append(run(xs))
        seq.append(run(xs))
        mdl.close()
        total = float(sum(range(1, n + 1)))
        want = [total] * 3 + [total - 6 + 100, total - 6 + 100 - 8 - 3]
        for (st, out), w in zip(seq[:5], want):
            assert st == 0 and np.allclose(out, w), (name, st, out, w)
        assert seq[5][0] != 0, name
        assert all(st == 0 and np.allclose(out, want[-1]) for st, out in seq[6:]), name
        results[name] = [st for st, _ in seq]
    if "ref" in results:
        assert results["mine"] == results["ref"]
