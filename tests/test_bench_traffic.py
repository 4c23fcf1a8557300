"""Provenance of the committed profile figures bench.py reports (CPU only):
roofline.traffic (the FETCH_SIZE / WRITE_SIZE figure) and the training
leg's in-step kernel times are used only when the profile row was measured
on this build's sources (decode kernels, training kernels); otherwise the
field is null and the line says why."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

ROW = "| traffic | stories110M | step | `{h}` | `k_decode_step` | 1024 | 1.0 | 1.0 | 475,901,952 | — | 484021082 |\n"


def test_sources_hash_covers_the_decode_sources():
    h = bench.decode_sources_hash()
    assert len(h) == 16 and int(h, 16) >= 0
    assert "pitorch_amd/csrc/ptmi_decode_step.hip" in bench.DECODE_SOURCES


def test_matching_sources_give_the_committed_figure(tmp_path):
    p = tmp_path / "traffic.md"
    p.write_text("# profile\n\n" + ROW.format(h=bench.decode_sources_hash()))
    assert bench.committed_traffic("step", "stories110M", path=str(p)) == (484021082, None)


def test_other_sources_give_null_with_the_reason(tmp_path):
    p = tmp_path / "traffic.md"
    p.write_text(ROW.format(h="0123456789abcdef"))
    value, note = bench.committed_traffic("step", "stories110M", path=str(p))
    assert value is None and "0123456789abcdef" in note and bench.decode_sources_hash() in note


def test_missing_row_or_file_gives_null(tmp_path):
    p = tmp_path / "traffic.md"
    p.write_text(ROW.format(h=bench.decode_sources_hash()))
    assert bench.committed_traffic("wo", "stories110M", path=str(p))[0] is None
    assert bench.committed_traffic("step", "stories110M", path=str(tmp_path / "none.md"))[0] is None


# The training step's in-step kernel times follow the same rule, keyed by
# the training kernels' sources.
IN_STEP = "| in-step | stories15M T256 | step | `{h}` | 18 | 612.5 | 802.4 |\n"


def test_in_step_times_need_the_training_sources():
    assert "pitorch_amd/csrc/ptmi_train.hip" in bench.TRAIN_SOURCES
    assert "pitorch_amd/csrc/ptmi_gemm.hip" in bench.TRAIN_SOURCES


def test_in_step_row_on_matching_sources(tmp_path):
    p = tmp_path / "train.md"
    p.write_text("# profile\n\n" + IN_STEP.format(h=bench.train_sources_hash()))
    got, note = bench.committed_in_step(path=str(p))
    assert note is None and got == {"steps": 18, "gemm_ms": 0.6125, "kernels_ms": 0.8024}


def test_in_step_row_on_other_sources_is_null(tmp_path):
    p = tmp_path / "train.md"
    p.write_text(IN_STEP.format(h="fedcba9876543210"))
    got, note = bench.committed_in_step(path=str(p))
    assert got is None and "fedcba9876543210" in note and bench.train_sources_hash() in note
    assert bench.committed_in_step(path=str(tmp_path / "none.md"))[0] is None
