"""After the rest of the GPU suite (collected before this file), the GPU's device error record is clear: no kernel
of a green run recorded a data error, including the persistent LSTM recurrence's bounded exchange polls. The
suite's own error cases (positions past a cache, ids out of range) are read and cleared by their tests."""
import pytest

pytestmark = pytest.mark.gpu


def test_device_error_record_is_clear_after_the_suite(gpu):
    from lokinfer_amd._lib import check_device_errors

    check_device_errors()
