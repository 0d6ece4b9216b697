"""Public BiGEMM entry point — delegates to backends (omniweave/ops/bigemm.py:24-73).

``backend`` is one of ``"hip"``, ``"auto"``, ``"reference"`` or ``"compile"``.

* ``"hip"``: the HIP kernels of libomniwave_amd.so; raises if unsupported for the inputs.
* ``"auto"``: ``"hip"`` when ``hip_is_supported`` says so, else the ``"reference"`` backend
  with the reason logged (omniweave/ops/dispatch.py:41-49).
* ``"reference"`` / ``"compile"``: this package ships no eager or compiled implementation of
  the operator.  A caller that has one (for example the upstream ``omniweave`` package, or a
  test oracle) registers it with ``register_backend``; calling an unregistered backend
  raises RuntimeError instead of silently running anything else.
"""

from __future__ import annotations

from collections.abc import Callable

from torch import Tensor

from omniwave_amd.dispatch import BACKENDS, select_backend
from omniwave_amd.routing import RoutePlan

_EXTERNAL: dict[str, Callable[..., Tensor]] = {}


def register_backend(name: str, fn: Callable[..., Tensor] | None) -> None:
    """Install (or with ``fn=None`` remove) the implementation behind ``"reference"`` or
    ``"compile"``.  ``fn`` takes the keyword arguments of ``bigemm`` minus ``backend``."""
    if name not in {"reference", "compile"}:
        raise ValueError(f"only 'reference' and 'compile' can be registered, got {name!r}")
    if fn is None:
        _EXTERNAL.pop(name, None)
    else:
        _EXTERNAL[name] = fn


def registered_backends() -> list[str]:
    return sorted(_EXTERNAL)


def bigemm(
    *,
    x: Tensor,
    plan: RoutePlan,
    a_u: Tensor,
    a_v: Tensor,
    a_o: Tensor,
    b_u: Tensor,
    b_v: Tensor,
    b_o: Tensor,
    gamma: Tensor,
    backend: str = "auto",
) -> Tensor:
    """Compute the BiGEMM residual delta of pre-normalised NHWC ``x`` ([B, H, W, C]).

    delta = gamma * A_o (SiLU(A_u T B_u) * (A_v T B_v)) B_o per routed tile
    (omniweave/ops/reference.py:120-173).
    """
    kwargs = dict(x=x, plan=plan, a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma)

    if backend == "hip":
        from omniwave_amd.hip import bigemm_delta_hip

        return bigemm_delta_hip(**kwargs)

    if backend in {"reference", "compile"}:
        fn = _EXTERNAL.get(backend)
        if fn is None:
            raise RuntimeError(
                f"backend {backend!r} is not registered: omniwave_amd implements the operator only "
                "with HIP kernels; use backend='hip' on a gfx950 GPU or register an implementation "
                "with omniwave_amd.bigemm.register_backend()"
            )
        return fn(**kwargs)

    if backend == "auto":
        from omniwave_amd.hip import hip_is_supported

        chosen, reason = select_backend(x, "auto", lambda t: hip_is_supported(t, plan, b_u))
        if chosen == "reference" and "reference" not in _EXTERNAL:
            raise RuntimeError(f"hip backend unsupported ({reason}) and no reference backend is registered")
        return bigemm(backend=chosen, **kwargs)

    raise ValueError(f"unknown backend: {backend!r}; expected one of {sorted(BACKENDS)}")
