"""hsn_amd: HSN's TBPTT window hot path (the top-k cell router, the sparse gated update with
its summary coupling, the backward recurrence and the carried-state gradient) as hand-written
HIP kernels for MI355X (gfx950), behind the reference's operator interface.

- :mod:`hsn_amd.window`: the whole-window path (route -> forward sweep -> backward) and its
  autograd node with the carried state.
- :mod:`hsn_amd.kernels.window`, :mod:`hsn_amd.kernels.ops`: drop-in mirrors of the reference's
  ``hsn.kernels.window`` and ``hsn.kernels.ops``.
- :mod:`hsn_amd.workload`: the benchmark's seeded synthetic windows and byte model.

Importing the package initialises no GPU and loads no library; the first operator call does,
and raises if ``libhsn_amd.so`` is missing or stale (``python -m hsn_amd.build``).
"""

__version__ = "0.1.0"
