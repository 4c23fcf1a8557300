"""bench.py's roofline.traffic provenance (CPU only): the committed
FETCH_SIZE / WRITE_SIZE figure is used only when the profile row was
measured on this build's decode sources; otherwise the field is null and
the line says why."""
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
