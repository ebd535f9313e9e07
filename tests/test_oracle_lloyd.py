"""The oracle's Lloyd update (update_centroids with the SplitHighestDistortion
repair) against the reference's own unit test of it
(fib-quant/src/lloyd.rs:364-402): samples (0,0), (1,0), (2,0), (10,0),
(10.1,0) on codewords (0,0), (10,0), (20,0) leave cell 2 empty; the
repair splits donor 0 (three samples, the highest distortion) along the
direction of its farthest sample, moving it below 1.0 and the new cell
above 1.0."""
import numpy as np
import pytest

from oracle import oracle as O


def test_reference_repair_case():
    samples = np.array([[0.0, 0.0], [1.0, 0.0], [2.0, 0.0], [10.0, 0.0], [10.1, 0.0]])
    start = np.array([[[0.0, 0.0], [10.0, 0.0], [20.0, 0.0]]])
    cb, mse, init = O.lloyd_refine(samples, start, 1)
    cb = cb[0].reshape(-1)
    assert cb[0] < 1.0 and cb[4] > 1.0                      # the reference's assertions
    assert cb[0] == 1.0 - 1.0e-6 and cb[4] == 1.0 + 1.0e-6   # centroid 1.0, farthest sample along +x
    assert cb[1] == 0.0 and cb[5] == 0.0
    assert cb[2] == (10.0 + 10.1) / 2                       # cell 1: mean of its two samples
    assert abs(init - (0.0 + 1.0 + 4.0 + 0.0 + (10.1 - 10.0) ** 2) / 5) == 0.0   # nearest distances, in order


def test_no_donor_is_an_error():
    with pytest.raises(O.OracleError):
        O.lloyd_refine(np.ones((6, 4)), np.array([[[1.0] * 4, [5.0] * 4]]), 2)
