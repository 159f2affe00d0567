"""The measurement helpers on the CPU: the PMC summaries that `profiles/` and
`bench.py` are built from (`gpa_amd.profiling`), on small synthetic counter
files whose answers are known, and the bench's reading of the committed
traffic table."""
import csv

import bench
from gpa_amd import profiling as pf

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(r)
    return str(path)


def _row(d, kernel, counter, value):
    return dict(Dispatch_Id=d, Kernel_Name=kernel, Counter_Name=counter, Counter_Value=value)


def test_timer_name_groups_state_kernels_by_key_width():
    assert pf.timer_name("gpa::gdn_chunk_bwd_mfma<gpa::bf16_t, 128>") == "gdn_chunk_bwd_mfma<bf16,128>"
    assert pf.timer_name("gpa::gdn_state_bwd_strip<128, true, true, false, true>") == "gdn_state_bwd_strip<128>"
    assert pf.timer_name("gpa::gdn_state_fwd_mfma_pack<256, true>") == "gdn_state_fwd_mfma_pack<256>"


def test_traffic_scales_each_counter_by_the_copy_calibration(tmp_path):
    """A copy of 1 MiB whose FETCH_SIZE reads 512 KiB and WRITE_SIZE 1024 KiB
    gives factors 2 and 1; a kernel whose counters read 100,000 and 50,000
    KiB per dispatch (two dispatches) then moves 200,000 KiB read and 50,000
    KiB written per dispatch (204.8 and 51.2 MB)."""
    copy = "__amd_rocclr_copyBuffer"
    kern = "void gpa::gdn_prep_mfma<gpa::bf16_t, 128, true>(gpa_gdn_problem, gpa_gdn_saved, int)"
    cf = _write(tmp_path / "cf.csv", [_row(0, copy, "FETCH_SIZE", 512.0)])
    cw = _write(tmp_path / "cw.csv", [_row(0, copy, "WRITE_SIZE", 1024.0)])
    f = _write(tmp_path / "f.csv", [_row(1, kern, "FETCH_SIZE", 1e5), _row(2, kern, "FETCH_SIZE", 1e5)])
    w = _write(tmp_path / "w.csv", [_row(1, kern, "WRITE_SIZE", 5e4), _row(2, kern, "WRITE_SIZE", 5e4)])
    text = pf.summarize_traffic(f, w, cf, cw, 1 << 20)
    assert "FETCH_SIZE x 2.000, WRITE_SIZE x 1.000" in text
    row = next(line for line in text.splitlines() if "gdn_prep_mfma" in line)
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[0] == "`gdn_prep_mfma<bf16,128,true>`" and cells[1] == "2"
    assert cells[2:] == ["100,000.0", "50,000.0", "204.8", "51.2"]


def test_stalls_are_shares_of_wave_cycles(tmp_path):
    kern = "void gpa::gdn_out_mfma<128>(gpa_gdn_problem, gpa_gdn_saved, gpa_operand, int)"
    first = [_row(0, kern, "SQ_WAVE_CYCLES", 1000.0)]
    first += [_row(0, kern, c, v) for c, v in zip(pf.STALL_PASSES[0][1:], (500, 250, 20, 300, 200, 50, 10))]
    second = [_row(0, kern, "SQ_LDS_BANK_CONFLICT", 30.0), _row(0, kern, "SQ_LDS_IDX_ACTIVE", 120.0),
              _row(0, kern, "SQ_WAVES", 8.0)]
    text = pf.summarize_stalls(_write(tmp_path / "a.csv", first), _write(tmp_path / "b.csv", second))
    row = next(line for line in text.splitlines() if "gdn_out_mfma" in line)
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[2:] == ["50 %", "25 %", "2 %", "30 %", "20 %", "5 %", "1 %", "25 %"]


def test_bench_reads_the_committed_traffic_table():
    """`roofline.traffic` of the dominant kernel comes from the committed PMC
    summary: read plus written MB per launch, in bytes."""
    got = bench._measured_traffic("gdn_chunk_bwd_mfma<bf16,128>")
    assert got is not None and 5e8 < got < 2e9
    assert bench._measured_traffic("no_such_kernel<1>") is None
