"""Host-side logic of the Python layer that needs no GPU: section starts of
the splatting API, feature widths of the fused perception, and the argument
checks that reject bad inputs before any kernel runs."""
import pytest
import torch

from npa_amd import perceive as PF
from npa_amd import splatting as SP


def test_splat_section_starts():
    s = SP._starts([3, 0, 5], "cpu")
    assert s.dtype == torch.int32 and s.tolist() == [0, 3, 3, 8]
    assert SP._starts([], "cpu").tolist() == [0]


def test_splat_sections_int_and_list():
    # torch.split semantics for an int block size: the last block is shorter
    x = torch.zeros(10, 2)
    calls = []
    orig = SP.Splat.apply
    try:
        SP.Splat.apply = staticmethod(lambda x, c, starts, *a: calls.append(starts.tolist()))
        SP.splat_particles_sections(x, torch.zeros(10, 3), 4)
        SP.splat_particles_sections(x, torch.zeros(10, 3), [6, 4])
        with pytest.raises(RuntimeError):
            SP.splat_particles_sections(x, torch.zeros(10, 3), [6, 3])
        with pytest.raises(RuntimeError):
            SP.splat_particles_sections(x, torch.zeros(10, 3), 0)
    finally:
        SP.Splat.apply = orig
    assert calls == [[0, 4, 8, 10], [0, 6, 10]]


def test_splat_rejects_bad_inputs():
    with pytest.raises(TypeError):
        SP.Splat.apply(torch.zeros(4, 2, dtype=torch.float64), torch.zeros(4, 3), torch.zeros(2, dtype=torch.int32),
                       8, 1.0, -1.0, 1.0, True, False, 0.1)
    with pytest.raises(TypeError):  # CPU tensors
        SP.Splat.apply(torch.zeros(4, 2), torch.zeros(4, 3), torch.zeros(2, dtype=torch.int32),
                       8, 1.0, -1.0, 1.0, True, False, 0.1)


def test_feature_width():
    C, D = 16, 3
    assert PF.feature_width(C, D, 0) == 2 * C
    assert PF.feature_width(C, D, PF.STATE_GRAD) == 2 * C + C * D
    assert PF.feature_width(C, D, PF.DENSITY_GRAD) == 2 * C + D
    assert PF.feature_width(C, D, PF.STATE_GRAD | PF.DENSITY_GRAD | PF.LOG_NORM_GRAD) == 2 * C + C * D + D


def test_perception_features_rejects_non_contiguous():
    s = torch.zeros(1, 4, 3)
    with pytest.raises(TypeError):
        PF.PerceptionFeatures.apply(s.transpose(1, 2).contiguous().transpose(1, 2), s, None, None, 2, 1.0, 1.0,
                                    4.0, 0)


def test_next_index_capacity():
    """The list's index-buffer policy: the last total plus 1/8 and 1024; a list
    that overflowed with a buffer smaller than its total keeps the margin, one
    that overflowed with room for its total (uneven slices) widens it, down to
    a margin of 1/2."""
    from npa_amd.sphops.sph_hip import next_index_capacity as nic
    assert nic(8000, 0, 10000, 3) == (8000 + 1000 + 1024, 3)
    assert nic(0, 0, 40, 3) == (1024, 3)
    # too small a buffer: the next one holds the total, margin unchanged
    cap, s = nic(1 << 20, 5, 1000, 3)
    assert s == 3 and cap >= 1 << 20
    # room for the total but rows did not fit: wider margin each time, to 1/2
    cap, s = nic(1 << 20, 5, 1 << 21, 3)
    assert s == 2 and cap == (1 << 20) + (1 << 18) + 1024
    assert nic(1 << 20, 5, 1 << 21, 2)[1] == 1
    assert nic(1 << 20, 5, 1 << 21, 1) == ((1 << 20) + (1 << 19) + 1024, 1)
    # totals above 2^31 stay exact (Python integers); the grid caps the buffer later
    assert nic(3 << 30, 0, 0, 3)[0] == (3 << 30) + (3 << 27) + 1024
