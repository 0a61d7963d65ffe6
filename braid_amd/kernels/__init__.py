"""Kernel entry points (``load_gdn``) over the gfx950 C-ABI library."""
