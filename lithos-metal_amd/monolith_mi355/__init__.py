"""monolith_mi355 — the MI355X (gfx950) backend for lithos-metal's token-loop decode layer.

Host-side mirror of the reference's operator API (``monolith/ops``, ``monolith/formats``) over hand-written HIP
kernels reached through the C ABI in ``include/lithos_mi355.h`` (``libmi355.so``).
"""

__version__ = "0.1.0"
