"""Write golden route-table vectors from the upstream reference (run in the build container only).

The reference's own tests check coverage and counts of the route plans but never their order
(``tests/test_routing.py``), so the order of ``_local_token_order`` at partial windows,
``_shifted_token_order`` (first-occurrence dedup), ``radix_order`` at levels >= 1 and
``_channel_order`` at levels >= 1 is pinned here by running the reference's
``omniweave/models/routing.py`` once and storing its outputs as data.

Only that one module file is loaded (its imports are torch/math/functools/dataclasses).
Output: ``tests/golden/routes.npz`` - for each case key ``<h>x<w>x<c>_g<g>_d<d>_<route><level>``
the arrays ``<key>/tok`` (int32 [Q_s*g]), ``<key>/ch`` (int32 [Q_c*d]) and
``<key>/meta`` (int32 [h, w, c, g, d, level, Q_s, Q_c]).

Usage: python tests/golden/make_route_fixtures.py [/root/reference]
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def cases() -> list[tuple[int, int, int, int, int, str, int]]:
    out = []
    # OmniWeave-T at 224 px and 384 px: every stage, every route/level the benchmarks use.
    for res in (224, 384):
        s = res // 4
        for i, (c, d) in enumerate(((128, 64), (256, 64), (512, 128), (1024, 128))):
            hw = s // (2 ** i)
            for route, level in (("local", 0), ("shifted", 0), ("radix", 0), ("radix", 1), ("radix", 2)):
                out.append((hw, hw, c, 16, d, route, level))
    # Shapes used by the reference's own tests.
    out += [
        (7, 7, 70, 16, 64, "radix", 1), (7, 7, 70, 16, 64, "local", 0),
        (8, 8, 128, 16, 64, "local", 0), (8, 8, 128, 16, 64, "shifted", 0),
        (8, 8, 128, 16, 64, "radix", 0), (8, 8, 128, 16, 64, "radix", 1),
        (4, 4, 4, 16, 4, "local", 0), (4, 4, 32, 16, 32, "local", 0),
        (8, 8, 16, 16, 8, "local", 0),
    ]
    # Odd shapes: partial windows on both axes, tiny grids, levels 0-3, ragged channels.
    for (h, w) in ((3, 3), (5, 9), (13, 6), (17, 17), (2, 11), (1, 1), (6, 6), (10, 10)):
        for route, level in (("local", 0), ("shifted", 0), ("radix", 0), ("radix", 1), ("radix", 2), ("radix", 3)):
            out.append((h, w, 72, 16, 16, route, level))
            out.append((h, w, 200, 16, 64, route, level))
    # Channel routing with ragged groups and rotations beyond the group count.
    for c, d, level in ((70, 64, 2), (130, 32, 5), (96, 32, 4), (64, 64, 1), (100, 16, 3)):
        out.append((4, 4, c, 16, d, "radix", level))
    # Larger radix levels (stride 256 inside 1024-token grids).
    out += [(32, 32, 64, 16, 64, "radix", 2), (32, 32, 64, 16, 64, "shifted", 0)]
    return out


def key(h, w, c, g, d, route, level) -> str:
    return f"{h}x{w}x{c}_g{g}_d{d}_{route}{level}"


def main() -> None:
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    path = ref / "omniweave" / "models" / "routing.py"
    spec = importlib.util.spec_from_file_location("_reference_routing", path)
    module = importlib.util.module_from_spec(spec)
    assert spec.loader is not None
    sys.modules[spec.name] = module  # dataclasses resolves annotations through sys.modules
    spec.loader.exec_module(module)
    arrays: dict[str, np.ndarray] = {}
    for (h, w, c, g, d, route, level) in cases():
        plan = module.build_route_plan(h, w, c, g, d, route, level)
        k = key(h, w, c, g, d, route, level)
        arrays[k + "/tok"] = plan.token_indices.reshape(-1).numpy().astype(np.int32)
        arrays[k + "/ch"] = plan.channel_indices.reshape(-1).numpy().astype(np.int32)
        q_s = plan.token_indices.shape[0]
        q_c = plan.channel_indices.shape[0]
        assert int(plan.token_mask.sum()) == h * w and int(plan.channel_mask.sum()) == c
        arrays[k + "/meta"] = np.array([h, w, c, g, d, level, q_s, q_c], dtype=np.int32)
    schedules = {depth: module.build_stage_schedule(depth) for depth in range(1, 12)}
    for depth, sched in schedules.items():
        arrays[f"schedule/{depth}"] = np.array(
            [[{"local": 0, "shifted": 1, "radix": 2}[r], lvl] for r, lvl in sched], dtype=np.int32
        )
    np.savez_compressed(HERE / "routes.npz", **arrays)
    print(f"wrote {len(cases())} route cases to {HERE / 'routes.npz'}")


if __name__ == "__main__":
    main()
