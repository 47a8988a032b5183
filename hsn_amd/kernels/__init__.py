"""The reference's kernel layer (``hsn.kernels``) on MI355X: :mod:`.window` mirrors
``hsn.kernels.window`` and :mod:`.ops` mirrors ``hsn.kernels.ops`` (the gated delta update and
the gather of the four-op ABI), both backed by ``libhsn_amd.so``."""
