"""profsum on synthetic rocprofv3 CSV: the decode-only launches are the
back-to-back ones, and FETCH/WRITE are scaled by the calibration copy."""
import csv

from amd_optimization_challenge_amd import profsum

TRACE_COLS = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X"]
PMC_COLS = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
DEC = "void mla::decode_h16_kernel<0, 0, true, 0>(mla::DecodeParams)"


def _write(path, cols, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(cols, r)))


def test_trace_splits_decode_only_from_in_call(tmp_path):
    rows, t = [], 0
    for _ in range(3):  # whole calls: flush, amax, decode (5 us), combine
        for name, d in [("fill", 50_000), ("mla::amax_kernel(x)", 4000), (DEC, 5000), ("mla::combine_kernel(x)", 3000)]:
            rows.append(("KERNEL_DISPATCH", name, t, t + d, 131072))
            t += d + 100
    for i in range(6):  # decode only, back to back: 2 warm-up (9 us) then 4 timed (7 us)
        d = 9000 if i < 2 else 7000
        rows.append(("KERNEL_DISPATCH", DEC, t, t + d, 131072))
        t += d + 100
    p = tmp_path / "p_kernel_trace.csv"
    _write(p, TRACE_COLS, rows)
    out = profsum.trace_summary(str(p), timed=4)
    line = [l for l in out.splitlines() if l.startswith("| 1 |")][0]
    cells = [c.strip() for c in line.split("|")]
    # one run of 6 back-to-back launches, the last 4 average 7 us; the three
    # in-call launches (each between an amax and a combine) average 5 us
    assert cells[4:6] == ["6", "7.00"], cells
    # launch period: (last end - first start) / 4 = (4 x 7000 + 3 x 100) / 4 ns
    assert cells[6] == f"{(4 * 7000 + 3 * 100) / 4 / 1e3:.2f}", cells
    incall = [l for l in out.splitlines() if l.startswith("| `decode_h16_kernel")][-1]
    assert [c.strip() for c in incall.split("|")][3:5] == ["3", "5.00"], incall


def test_pmc_scaled_by_calibration_copy(tmp_path):
    fetch = [(1, "__amd_rocclr_copyBuffer", 1, "FETCH_SIZE", 131072.0), (2, DEC, 7, "FETCH_SIZE", 1000.0),
             (3, DEC, 7, "FETCH_SIZE", 3000.0)]
    write = [(1, "__amd_rocclr_copyBuffer", 1, "WRITE_SIZE", 262144.0), (2, DEC, 7, "WRITE_SIZE", 100.0),
             (3, DEC, 7, "WRITE_SIZE", 300.0)]
    _write(tmp_path / "f.csv", PMC_COLS, fetch)
    _write(tmp_path / "w.csv", PMC_COLS, write)
    out = profsum.pmc_summary(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"))
    assert "FETCH_SIZE x 2.000, WRITE_SIZE x 1.000" in out
    # mean fetch 2000 KiB x 2 + mean write 200 KiB x 1, in bytes
    assert f"traffic.launch1={(2000 * 2 + 200) * 1024}" in out


def test_pmc_runs_split_by_set_up_kernels(tmp_path):
    """Two runs of one kernel (same grid), separated by a re-layout copy, stay
    two rows; flush fills between launches do not split a run."""
    def rows(counter, vals):
        out, d = [(1, "__amd_rocclr_copyBuffer", 1, counter, 131072.0 if counter == "FETCH_SIZE" else 262144.0)], 2
        for i, v in enumerate(vals):
            if i == 2:
                out.append((d, "elementwise_kernel copy", 9, counter, 5.0))
                d += 1
            out.append((d, "FillFunctor<unsigned char>", 9, counter, 1.0))
            out.append((d + 1, DEC, 7, counter, v))
            d += 2
        return out
    _write(tmp_path / "f.csv", PMC_COLS, rows("FETCH_SIZE", [1000.0, 1000.0, 500.0, 500.0]))
    _write(tmp_path / "w.csv", PMC_COLS, rows("WRITE_SIZE", [10.0, 10.0, 10.0, 10.0]))
    out = profsum.pmc_summary(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"))
    assert f"traffic.launch1={(2000 + 10) * 1024}" in out and f"traffic.launch2={(1000 + 10) * 1024}" in out


def test_calls_groups_whole_calls_and_skips_decode_only_runs(tmp_path):
    """Whole calls (flush, then amax, quant, one decode, combine) are grouped
    by their kernels; a decode-only run followed by a combine is not a call."""
    rows, t = [], 0
    for i in range(3):
        for name, d, gap in [("fill", 50_000, 100), ("mla::amax_kernel(x)", 4000 + 1000 * i, 200),
                             ("mla::quant_fp8_kernel(x)", 5000, 300), (DEC, 60_000, 400),
                             ("mla::combine_kernel(x)", 8000, 100)]:
            rows.append(("KERNEL_DISPATCH", name, t, t + d, 4096))
            t += d + gap
    for name, d in [(DEC, 7000), (DEC, 7000), ("mla::combine_kernel(x)", 3000)]:
        rows.append(("KERNEL_DISPATCH", name, t, t + d, 4096))
        t += d + 100
    p = tmp_path / "p_kernel_trace.csv"
    _write(p, TRACE_COLS, rows)
    out = profsum.calls_summary(str(p))
    assert out.count(" calls") == 1 and out.startswith("3 calls"), out
    amax = [l for l in out.splitlines() if l.startswith("| 1 |")][0]
    assert [c.strip() for c in amax.split("|")][4:7] == ["5.00", "4.00", "-"], amax
    dec = [l for l in out.splitlines() if l.startswith("| 3 |")][0]
    assert [c.strip() for c in dec.split("|")][4:7] == ["60.00", "60.00", "0.30"], dec
    # span: amax start to combine end = amax + 200 + 5000 + 300 + 60000 + 400 + 8000 (median amax 5000)
    assert f"median {(5000 + 200 + 5000 + 300 + 60000 + 400 + 8000) / 1e3:.2f} us" in out, out
