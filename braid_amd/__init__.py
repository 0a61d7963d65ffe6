"""braid_amd: the Gated DeltaNet mixer hot path of braid, built for MI355X (gfx950).

``braid_amd.kernels.loader.load_gdn()`` is the drop-in for
``braid.kernels.loader.load_gdn()``; the kernels are hand-written HIP in
``braid_amd/csrc`` behind the C ABI of ``include/braid_gdn.h``.
"""
__version__ = "0.1.0"
