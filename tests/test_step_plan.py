"""The one-kernel decode step's launch plan (CPU only: pure host arithmetic
behind ptmi_decode_step_plan, no device call).

The step runs one workgroup per compute unit, all resident at once, and
gives every attention unit (head, chunk of positions) a workgroup of its
own; anything else takes the multi-kernel step.  These cases pin that
decision: the stories shapes on a full MI355X (256 compute units), a
partitioned device too small for the units, a kernel that would not fit
one workgroup per unit, the shapes the kernel does not take, and the
wrapped-unit shape of 48 heads (384 units, more than the workgroups: a
head's chunk-0 unit could then wait behind another merge on its own
workgroup, so it must fall back)."""
import pytest

import pitorch_amd as pa

OK, SHAPE, RESIDENT = 0, 1, 2


@pytest.mark.parametrize("name, units", [("stories15M", 48), ("stories42M", 64), ("stories110M", 96)])
def test_stories_shapes_run_as_one_kernel_on_a_full_device(name, units):
    reason, grid, n_units = pa.decode_step_plan(pa.STORIES[name], 256, 1)
    assert (reason, grid, n_units) == (OK, 256, units)


def test_grid_is_one_workgroup_per_compute_unit_up_to_512():
    assert pa.decode_step_plan(pa.STORIES["stories110M"], 304, 1)[:2] == (OK, 304)
    assert pa.decode_step_plan(pa.STORIES["stories110M"], 1024, 2)[:2] == (OK, 512)


def test_too_few_compute_units_for_the_attention_units_falls_back():
    # 96 units of stories110M need 96 workgroups; a 64-CU partition has 64
    assert pa.decode_step_plan(pa.STORIES["stories110M"], 96, 1)[0] == OK
    assert pa.decode_step_plan(pa.STORIES["stories110M"], 95, 1)[0] == RESIDENT
    assert pa.decode_step_plan(pa.STORIES["stories110M"], 64, 1)[0] == RESIDENT


def test_kernel_that_does_not_fit_a_compute_unit_falls_back():
    assert pa.decode_step_plan(pa.STORIES["stories110M"], 256, 0)[0] == RESIDENT
    assert pa.decode_step_plan(pa.STORIES["stories110M"], 0, 1)[0] == RESIDENT


def test_wrapped_attention_units_fall_back():
    # dim 768 as 48 heads of 16, 1024 positions: 48 * 8 = 384 units > 256
    reason, grid, units = pa.decode_step_plan((768, 2048, 1, 48, 48, 512, 1024), 256, 1)
    assert (reason, units) == (RESIDENT, 384)


@pytest.mark.parametrize("cfg", [
    (256, 512, 2, 2, 2, 512, 64),         # head_dim 128: the kernel takes <= 64
    (4096, 1024, 1, 64, 64, 512, 64),     # dim past 2048
    (288, 770, 1, 6, 6, 512, 64),         # hidden not a multiple of 4
    (768, 2048, 1, 12, 12, 512, 4096),    # 4096 positions: more than 8 units of <= 128 per head
])
def test_unsupported_shapes_take_the_multi_kernel_step(cfg):
    assert pa.decode_step_plan(cfg, 256, 1)[0] == SHAPE


def test_bad_shape_is_an_argument_error():
    with pytest.raises(pa.PtmiError):
        pa.decode_step_plan((768, 2048, 1, 5, 5, 512, 64), 256, 1)   # dim % heads
