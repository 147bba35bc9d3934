"""bench.py's contract pieces that need no GPU: the one-GPU refusal and the
measured-traffic lookup the roofline objects carry."""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.join(os.path.dirname(__file__), "..")


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in r.stderr and r.stdout == ""


def test_roofline_traffic_is_tied_to_the_code_object(tmp_path):
    """A traffic line counts only for the code object it was measured on."""
    b = _bench()
    h = b.code_object_hash("dsmoe_up_rows")
    assert h is not None and len(h) == 16
    assert b.code_object_hash("dsmoe_gu_grouped") != h
    f = tmp_path / "moe_decode_c2_traffic.txt"
    f.write_text(f"traffic kernel=dsmoe_up_rows config=c2 path=staged bytes=123 code_object={h}\n"
                 f"traffic kernel=dsmoe_dn_rows config=c2 path=staged bytes=456 code_object=0123456789abcdef\n")
    assert b.measured_traffic("dsmoe_up_rows", "c2", "staged", str(tmp_path)) == 123
    assert b.measured_traffic("dsmoe_dn_rows", "c2", "staged", str(tmp_path)) is None  # stale
    assert b.measured_traffic("dsmoe_prep", "c2", "staged", str(tmp_path)) is None  # not measured


def test_committed_traffic_summaries_carry_the_keys_the_bench_reads():
    """The bench line's roofline.traffic comes from profiles/: the committed
    summaries must hold lines under exactly the kernel, config and path names
    the bench looks up (decode c2 on the row-streaming path, prefill c5 on the
    grouped path), whatever build they were measured on."""
    b = _bench()
    want = [("dsmoe_up_rows", "c2", "staged"), ("dsmoe_dn_rows", "c2", "staged"),
            ("dsmoe_gu_grouped", "c5", "grouped"), ("dsmoe_dn_grouped", "c5", "grouped")]
    keys = set()
    for kind, cfg in (("decode", "c2"), ("prefill", "c5")):
        for line in open(os.path.join(ROOT, "profiles", f"moe_{kind}_{cfg}_traffic.txt")):
            if line.startswith("traffic "):
                kv = dict(t.split("=", 1) for t in line.split()[1:])
                keys.add((kv["kernel"], kv["config"], kv["path"]))
    for k in want:
        assert k in keys, k
    assert b.STAGE_KERNEL["up"] == "dsmoe_up_rows" and b.PREFILL_KERNEL["gu_grouped"] == "dsmoe_gu_grouped"


def test_cpu_baseline_value_is_the_all_core_run():
    """cpu_baseline.value is the oracle at every host core (os.cpu_count()),
    with the 1-thread figure as a side field, on the small config."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "deepseek-rs_amd"))
    from dsmoe import configs as C
    b = _bench()
    case = C.CASES["c1"]
    w = C.make_weights(case, device="cpu")
    hw = b.host_weights(w)
    xs = [C.make_x(case, T=1, step=s, device="cpu") for s in range(2)]
    cpu = b.cpu_main(case, hw, xs, 0.2)
    assert cpu["cores"] == os.cpu_count() and cpu["kind"] == "port" and cpu["unit"] == "tokens/s"
    assert cpu["value"] > 0 and cpu["value_1_thread"] > 0
    assert f"{os.cpu_count()} threads" in cpu["sample"] and "1 thread" in cpu["sample_1_thread"]
    pair = b.cpu_pair(case, hw, xs, 0.1, None, None)
    assert pair["threads"] == os.cpu_count() and pair["tokens_per_s_1_thread"] > 0
    assert np.isfinite(pair["tokens_per_s"])


def test_profile_summary_busy_fractions():
    """derived() turns one run's counter medians into busy fractions:
    a kernel whose 256 CUs each issue VALU work on every one of its cycles
    (GRBM_GUI_ACTIVE summed over 8 XCDs) is valu_busy 1.0; the matrix-core
    share is per SIMD (1024 of them); the TA share is a plain ratio."""
    sys.path.insert(0, os.path.join(ROOT, "deepseek-rs_amd"))
    import profile_summary as P
    cyc = 1000.0
    d = P.derived({"GRBM_GUI_ACTIVE": 8 * cyc, "SQ_ACTIVE_INST_VALU": 256 * cyc, "SQ_ACTIVE_INST_LDS": 64 * cyc,
                   "SQ_LDS_BANK_CONFLICT": 128 * cyc, "SQ_VALU_MFMA_BUSY_CYCLES": 512 * cyc,
                   "SQ_VALU_MFMA_COEXEC_CYCLES": 128 * cyc, "TA_TA_BUSY": 400.0,
                   "TA_ADDR_STALLED_BY_TC_CYCLES": 100.0})
    assert d == {"valu_busy": 1.0, "lds_busy": 0.25, "lds_bank_conflict": 0.5, "mfma_busy": 0.5,
                 "mfma_coexec": 0.25, "ta_stalled_by_tc": 0.25}
    # without the clock only the ratios that need none are formed
    assert P.derived({"SQ_ACTIVE_INST_VALU": 1.0, "TA_TA_BUSY": 2.0, "TA_ADDR_STALLED_BY_TC_CYCLES": 1.0}) == \
        {"ta_stalled_by_tc": 0.5}
