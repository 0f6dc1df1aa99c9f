"""Host-side workspace sizing of the packed linear (no GPU): a run of growing batch sizes
replaces the workspace O(log n) times, and the buffers kept alive for captured graphs stay
smaller together than the current one."""
import importlib

import torch

from conftest import PKG


class _Owner:
    def __init__(self):
        self._ws = None
        self._ws_retired = []
        self.device = torch.device("cpu")


def test_workspace_growth_is_geometric():
    pl = importlib.import_module(PKG + ".packed_linear")
    owner = _Owner()
    # prefill lengths 1..4096 on a 4096-wide linear: ~16 KB of workspace per row
    needs = [16384 * b + 1024 for b in range(1, 4097)]
    for need in needs:
        ws = pl._grow_workspace(owner, need)
        assert ws.numel() >= need
        assert ws.numel() & (ws.numel() - 1) == 0      # a power of two
        assert ws.numel() < 2 * need or ws.numel() == 256
    assert len(owner._ws_retired) <= (needs[-1]).bit_length()
    assert sum(w.numel() for w in owner._ws_retired) < owner._ws.numel()
    # a smaller request keeps the current buffer
    cur = owner._ws
    assert pl._grow_workspace(owner, 100) is cur
    assert pl._ws_size(1) == 256 and pl._ws_size(256) == 256 and pl._ws_size(257) == 512
