"""CPU tests of the rocprofv3 report extractor (flash-attention-cuda_amd/profile).

The capture runs on the GPU box; these guard the parsing and the arithmetic
on synthetic rocprofv3 CSVs, as the reference's tests/test_ncu_extract.py
guards its Nsight parser. No GPU needed.
"""

import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "flash-attention-cuda_amd", "profile"))

import rocprof_extract as rx  # noqa: E402


@pytest.mark.parametrize("raw,expected", [
    ("void fa::(anonymous namespace)::prefill_kernel<true, false>(_Float16 const*, int)",
     "prefill_kernel<true, false>"),
    ("void fa::(anonymous namespace)::prefill_kernel<false, false>(_Float16 const*, int)",
     "prefill_kernel<false, false>"),
    ("void fa::(anonymous namespace)::decode_merge_kernel<false>(float const*, int)",
     "decode_merge_kernel<false>"),
    ("fa::(anonymous namespace)::decode_split_kernel(_Float16 const*)", "decode_split_kernel"),
    ("void at::native::foo<int, (anonymous namespace)::bar<2> >(int)",
     "foo<int, bar<2> >"),
    ("__amd_rocclr_copyBuffer", "__amd_rocclr_copyBuffer"),
])
def test_short_kernel_name(raw, expected):
    assert rx.short_kernel_name(raw) == expected


def test_mangled_names_are_demangled_and_instantiations_stay_apart():
    causal = rx.short_kernel_name("_ZN2fa12_GLOBAL__N_114prefill_kernelILb1ELb0EEEvPKDF16_S3_S3_Pviiifb")
    full = rx.short_kernel_name("_ZN2fa12_GLOBAL__N_114prefill_kernelILb0ELb0EEEvPKDF16_S3_S3_Pviiifb")
    assert causal == "prefill_kernel<true, false>" and full == "prefill_kernel<false, false>"
    # The head size is the first template argument of the current kernels.
    d128 = rx.short_kernel_name(
        "_ZN2fa12_GLOBAL__N_114prefill_kernelILi128ELb1ELb0EEEvPKDF16_S3_S3_Pviiifb")
    assert d128 == "prefill_kernel<128, true, false>"
    assert rx.short_kernel_name(
        "_ZN2fa12_GLOBAL__N_119decode_group_kernelEPKDF16_S2_S2_PKiPfS5_iiiiiiiif") == \
        "decode_group_kernel"
    assert rx.short_kernel_name("_ZN2fa12_GLOBAL__N_116decode_bh_kernelILb0EEEvPKDF16_") == \
        "decode_bh_kernel<false>"
    assert rx._demangle_nested("_ZN1a1bILi8ELin3EEEv") == "a::b<8, -3>()"
    assert rx._demangle_nested("_Z3fooIdEv") is None  # not a literal argument


STATS = '''"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"
"void fa::(anonymous namespace)::prefill_kernel<64, true, false>(_Float16 const*)",25,1250000,50000.0,90.0,48000,52000,100.0
"__amd_rocclr_copyBuffer",2,20000,10000.0,10.0,9000,11000,5.0
'''

COUNTERS_HDR = ('"Correlation_Id","Dispatch_Id","Agent_Id","Queue_Id","Process_Id","Thread_Id",'
                '"Grid_Size","Kernel_Id","Kernel_Name","Workgroup_Size","LDS_Block_Size",'
                '"Scratch_Size","VGPR_Count","Accum_VGPR_Count","SGPR_Count","Counter_Name",'
                '"Counter_Value","Start_Timestamp","End_Timestamp"\n')


def _counter_rows(kernel, counter, values):
    return "".join(f'{i},{i},"Agent 1",1,1,1,64,1,"{kernel}",64,0,0,1,0,1,"{counter}",{v},0,1\n'
                   for i, v in enumerate(values))


def _write(path, text):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", encoding="utf-8") as handle:
        handle.write(text)


PK = "void fa::(anonymous namespace)::prefill_kernel<64, true, false>(_Float16 const*)"


def _tree(root):
    # Calibration: the copy counts 524288 KiB fetched (half of 1 GiB) and
    # 1048576 KiB written per launch -> 2048 and 1024 bytes per KiB.
    _write(f"{root}/copy_1g/trace/run_kernel_stats.csv", STATS)
    _write(f"{root}/copy_1g/fetch/run_counter_collection.csv",
           COUNTERS_HDR + _counter_rows("__amd_rocclr_copyBuffer", "FETCH_SIZE", [524288, 524288]))
    _write(f"{root}/copy_1g/write/run_counter_collection.csv",
           COUNTERS_HDR + _counter_rows("__amd_rocclr_copyBuffer", "WRITE_SIZE", [1048576]))
    _write(f"{root}/prefill_c3/trace/run_kernel_stats.csv", STATS)
    _write(f"{root}/prefill_c3/fetch/run_counter_collection.csv",
           COUNTERS_HDR + _counter_rows(PK, "FETCH_SIZE", [14000, 16000]))
    _write(f"{root}/prefill_c3/write/run_counter_collection.csv",
           COUNTERS_HDR + _counter_rows(PK, "WRITE_SIZE", [7168]))
    _write(f"{root}/prefill_c3/sq/run_counter_collection.csv",
           COUNTERS_HDR + _counter_rows(PK, "MfmaUtil", [30.0, 32.0])
           + _counter_rows(PK, "MfmaFlopsF16", [3.0e10])
           + _counter_rows(PK, "LdsBankConflict", [0.01])
           + _counter_rows(PK, "OccupancyPercent", [25.0]))


def test_parsers(tmp_path):
    root = str(tmp_path)
    _tree(root)
    stats = rx.read_kernel_stats(f"{root}/prefill_c3/trace/run_kernel_stats.csv")
    assert stats["prefill_kernel<64, true, false>"]["calls"] == 25
    assert stats["prefill_kernel<64, true, false>"]["avg_us"] == 50.0
    counters = rx.read_counters(f"{root}/prefill_c3/fetch/run_counter_collection.csv")
    assert counters["prefill_kernel<64, true, false>"]["FETCH_SIZE"] == 15000.0  # mean of dispatches
    assert rx.calibration(root) == (2048.0, 1024.0)


def test_analyse_and_render(tmp_path):
    root = str(tmp_path)
    _tree(root)
    report = rx.analyse(root)
    w = report["workloads"]["prefill_c3"]
    k = w["kernels"]["prefill_kernel<64, true, false>"]
    assert k["read_bytes"] == 15000.0 * 2048 and k["write_bytes"] == 7168 * 1024
    assert k["mfma_util_pct"] == 31.0 and k["occupancy_pct"] == 25.0
    main = w["main"]
    assert main["kernel"] == "prefill_kernel<64, true, false>"
    # config 3: 30,064,771,072 FLOP in 50 us
    assert abs(main["rate"] - 30064771072.0 / 50e-6) < 1.0
    assert abs(main["frac"] - main["rate"] / 2516.6e12) < 1e-12
    text = rx.render(report, "bash profile_rocprof.sh")
    assert "prefill_kernel<64, true, false>" in text and "bash profile_rocprof.sh" in text
    assert f"{100 * main['frac']:.1f} %" in text
    assert "31.0 %" in text and "30.72 MB" in text  # 15000 KiB x 2048 B/KiB
    # Workloads without traces are left out, not rendered empty.
    assert "decode_c5" not in text
    paths = rx.write_split(report, str(tmp_path / "split"), "cmd")
    names = sorted(os.path.basename(p) for p in paths)
    assert names == ["copy_1g__amd_rocclr_copyBuffer.md", "prefill_c3__prefill_kernel.md"]
    body = open(tmp_path / "split" / "prefill_c3__prefill_kernel.md", encoding="utf-8").read()
    traffic = [ln for ln in body.splitlines() if ln.startswith("traffic_bytes_per_launch:")]
    assert traffic == [f"traffic_bytes_per_launch: {15000 * 2048 + 7168 * 1024}"]


def test_bench_runs_pair_trace_and_events(tmp_path):
    root = str(tmp_path)
    _write(f"{root}/bench_prefill/trace/run_kernel_stats.csv", STATS)
    _write(f"{root}/bench_prefill/trace.log",
           'timing ...\n{"value": 600.0, "roofline": {"kernel": "prefill_kernel<causal=true>", '
           '"kernel_ms": 0.0495, "achieved": 607.4, "unit": "TFLOP/s"}}\n')
    runs = rx.bench_runs(root)
    assert runs["prefill"]["kernel"] == "prefill_kernel<64, true, false>"
    assert runs["prefill"]["trace_avg_us"] == 50.0
    assert abs(runs["prefill"]["bench_event_us"] - 49.5) < 1e-9
    assert "bench_decode" not in runs and "decode" not in runs


def test_missing_counter_column_is_an_error(tmp_path):
    bad = tmp_path / "c.csv"
    bad.write_text('"a","b"\n1,2\n', encoding="utf-8")
    with pytest.raises(SystemExit):
        rx.read_counters(str(bad))


def test_main_refuses_an_empty_root(tmp_path):
    with pytest.raises(SystemExit):
        rx.main(["--root", str(tmp_path), "--out", str(tmp_path / "r.md")])
