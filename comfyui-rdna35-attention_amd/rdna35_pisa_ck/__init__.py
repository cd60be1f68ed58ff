"""The reference's native module name, bound to the gfx950 implementation.

Callers of the reference import its native PISA package by name
(``import rdna35_pisa_ck``: rdna35_block_attention/pisa_attention.py:216,
generic_pisa.py:121, pisa_patch.py:226).  Importing this package gives them
the ``mi355x_pisa`` module itself - the same ``forward``,
``forward_spatial_bhtd``, ``block_stats_hyd``, ``prepare``, ``build_info``,
``capabilities``, ``clear_compile_cache`` and ``_C`` surface - so such code
runs on the HIP kernels unchanged.  ``build_info()["architecture"]`` reports
gfx950: callers that insist on gfx1151 see a clear mismatch instead of a
silent substitution.
"""
import sys

import mi355x_pisa as _implementation

sys.modules[__name__] = _implementation
