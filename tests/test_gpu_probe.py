"""The streaming-read probe (tri_stream_read, a measurement aid of the bench) runs through the C ABI
for every launch shape it accepts, reads ragged record counts without writing anything, and rejects
shapes outside its contract."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("records", [1, 37, 512])
def test_stream_read_shapes(module, records):
    buf = torch.full((records * 8192,), 7, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    for waves, wpg, depth in ((1, 1, 1), (64, 1, 2), (64, 2, 3), (1024, 4, 2), (4096, 4, 3)):
        module.stream_read(buf, waves, wpg, depth, sink)
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    assert bool((buf == 7).all())


def test_stream_read_rejects(module):
    buf = torch.zeros(8192, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="waves_per_group"):
        module.stream_read(buf, 64, 3, 1, sink)
    with pytest.raises(RuntimeError, match="depth"):
        module.stream_read(buf, 64, 1, 4, sink)
    with pytest.raises(RuntimeError, match="positive"):
        module.stream_read(buf[:100], 64, 1, 1, sink)
