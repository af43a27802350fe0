"""``turboquant.quantizer`` of the reference's module layout
(turboquant/quantizer.py): TurboQuantMSE / TurboQuantProd and the bit
packing helpers under the reference's private names (its tests import
``_pack_bits`` / ``_unpack_bits``), from ``turboquant_amd.algorithm``."""
from .algorithm import TurboQuantMSE, TurboQuantProd
from .algorithm import pack_bits as _pack_bits
from .algorithm import unpack_bits as _unpack_bits

__all__ = ["TurboQuantMSE", "TurboQuantProd", "_pack_bits", "_unpack_bits"]
