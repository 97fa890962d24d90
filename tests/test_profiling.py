"""The rocprofv3 summary tool's traffic calibration (CPU only: synthetic counter CSVs).

FETCH_SIZE / WRITE_SIZE readings are scaled by what the same counters read for the
256 MiB calibration copy that `bench.py --profile` runs. An input recipe may launch
the copy's kernel on larger or smaller tensors too; the copy is told apart by its grid.
"""

import csv

from evograd_amd import profiling

FIELDS = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value",
          "Start_Timestamp", "End_Timestamp"]
COPY = "void at::native::vectorized_elementwise_kernel<4, at::native::AUnaryFunctor<float, " \
       "float, float, at::native::binary_internal::MulFunctor<float> > >"


def _write(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (name, grid, kib) in enumerate(rows):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Grid_Size": grid,
                        "Counter_Name": counter, "Counter_Value": kib,
                        "Start_Timestamp": 0, "End_Timestamp": 1000})


def test_traffic_calibrates_on_the_copy_grid_not_the_largest_reading(tmp_path):
    copy_kib = profiling.COPY_BYTES / 1024
    # FETCH_SIZE reads half the copy's bytes on this part (x2 calibration), WRITE_SIZE
    # all of them; a recipe scaling an 8x larger tensor with the same kernel comes first
    fetch = [(COPY, profiling.COPY_GRID * 8, 8 * copy_kib / 2),
             ("eg::my_kernel", 4096, 1000.0),
             ("eg::my_kernel", 4096, 1002.0),
             (COPY, profiling.COPY_GRID, copy_kib / 2)]
    write = [(COPY, profiling.COPY_GRID * 8, 8 * copy_kib),
             ("eg::my_kernel", 4096, 500.0),
             ("eg::my_kernel", 4096, 500.0),
             (COPY, profiling.COPY_GRID, copy_kib)]
    _write(tmp_path / "f.csv", "FETCH_SIZE", fetch)
    _write(tmp_path / "w.csv", "WRITE_SIZE", write)
    e = profiling.traffic(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), "my_kernel", "k")
    assert e["key"] == "k"
    assert abs(e["copy_calibration"]["fetch_scale"] - 2.0) < 1e-12
    assert abs(e["copy_calibration"]["write_scale"] - 1.0) < 1e-12
    # the kernel's median reading (1001 KiB fetched, 500 KiB written), scaled
    assert e["fetch_bytes_per_launch"] == round(1001.0 * 1024 * 2)
    assert e["write_bytes_per_launch"] == 500 * 1024
    assert e["hbm_bytes_per_launch"] == e["fetch_bytes_per_launch"] + e["write_bytes_per_launch"]
