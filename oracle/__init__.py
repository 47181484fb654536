"""CPU oracle for the uTTT hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in PyTorch on the CPU, the arithmetic of the reference
uTTT hot path (``model/uttt_layer.py`` and ``model/uttt_model.py`` of
Phova/uTTTCompanion).  It exists to *check* the HIP implementation in
``utttcompanion_amd``; it is never the thing measured or shipped.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package must not import it, and the
product path fails loudly when its HIP library is missing instead of falling
back to anything in here.

Pinning status of each function (what independent check fixes its values) is
recorded in the docstring of each function in ``uttt_math``; the tests under
``tests/test_oracle_*.py`` hold those checks.
"""

from . import uttt_math  # noqa: F401
