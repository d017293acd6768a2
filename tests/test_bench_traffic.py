"""The bench's reading of rocprofv3 counter CSVs for the roofline's traffic:
the copy of known size is the copy dispatch with the largest grid, the
attention is the tiled verify kernel, and a CSV missing either is an error
(the bench then reports its stored figure and says why)."""
import csv

import pytest

import bench

HEADER = ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
TILED = "void specdec::attention_bf16_kernel<1, 16, true, false>(specdec::AttnArgs)"


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(HEADER)
        w.writerows(rows)


def test_copy_of_largest_grid_and_tiled_attention_are_averaged(tmp_path):
    p = tmp_path / "f_counter_collection.csv"
    _write(p, [
        ["__amd_rocclr_copyBuffer", "512", "FETCH_SIZE", "3.0"],          # a small staging copy
        ["__amd_rocclr_copyBuffer", "131072", "FETCH_SIZE", "131090.0"],
        ["__amd_rocclr_copyBuffer", "131072", "FETCH_SIZE", "131082.0"],
        [TILED, "262144", "FETCH_SIZE", "132000.0"],
        [TILED, "262144", "FETCH_SIZE", "132100.0"],
        ["void specdec::attention_bf16_kernel<1, 4, false, false>(specdec::AttnArgs)", "2048", "FETCH_SIZE", "9.0"],
        [TILED, "262144", "WRITE_SIZE", "160.0"],                          # another counter: ignored
    ])
    copy_kib, attn_kib, n = bench._counter_means(str(p), "FETCH_SIZE")
    assert (copy_kib, attn_kib, n) == (131086.0, 132050.0, 2)
    # FETCH_SIZE reads half the bytes a copy moves: the scale is about 2
    assert bench.COPY_BYTES / (copy_kib * 1024) == pytest.approx(2.0, rel=1e-3)


@pytest.mark.parametrize("drop", ["copy", "attention"])
def test_a_csv_without_the_copy_or_the_attention_is_refused(tmp_path, drop):
    p = tmp_path / "w_counter_collection.csv"
    rows = [["__amd_rocclr_copyBuffer", "131072", "WRITE_SIZE", "262144.0"], [TILED, "262144", "WRITE_SIZE", "160.0"]]
    _write(p, [r for r in rows if (drop == "copy") != ("copyBuffer" in r[0])])
    with pytest.raises(RuntimeError, match=f"no {drop} dispatch"):
        bench._counter_means(str(p), "WRITE_SIZE")
