"""GPU: the workgroup hand-off of grid_sync.h (lq8_bench_grid_sync): for
every synchronisation kind, at one and two workgroups per CU, every value
exchanged between workgroups across a grid-wide synchronisation is read
back exactly (no stale cache line), and no bounded wait gives up."""
import pytest

import lq8

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("per_cu", [1, 2])
def test_grid_sync_exchange_is_coherent(ctx, kind, per_cu):
    nwg = 256 * per_cu
    us, bad, gave_up = lq8.bench_grid_sync(ctx, kind, nwg, 200)
    print(f"kind {kind}, {nwg} workgroups: {us:.2f} us per synchronisation")
    assert gave_up == 0
    assert bad == 0
    assert us > 0
