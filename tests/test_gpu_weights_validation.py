"""GPU-box test of the safetensors reader's header checks (the format of
safetensors.cpp:81-200): a header whose shape or offsets are not
non-negative integers, or whose element count overflows 64 bits, is
rejected with an error naming the tensor, before any tensor is built from
it. Each file holds one F32 entry of 24 data bytes."""
import json
import struct

import pytest

import sdhip

pytestmark = pytest.mark.gpu


def _file(tmp_path, shape, offsets=(0, 24)):
    hdr = json.dumps({"w": {"dtype": "F32", "shape": shape, "data_offsets": list(offsets)}}).encode()
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(24))
    return p


@pytest.mark.parametrize("shape,offsets,msg", [
    ([-2, -3], (0, 24), "bad dimension"),                    # negative dims whose product is right
    ([2.5, 2.4], (0, 24), "bad dimension"),                  # non-integral
    ([1 << 40, 1 << 40, 1 << 40], (0, 24), "overflows"),     # product past 2^63
    ([2, 3], (-8, 24), "bad offset"),
    ([2, 3], (0, 28), "bad offsets"),                        # past the end of the data
    ([2, 4], (0, 24), "size mismatch"),
])
def test_malformed_header_rejected(tmp_path, shape, offsets, msg):
    with pytest.raises(sdhip.SdhError) as e:
        sdhip.ZImage.load(_file(tmp_path, shape, offsets))
    assert msg in str(e.value) and "w" in str(e.value), str(e.value)
