"""The draft model around the INT8 tier (mirror of reference ksdraft/model/__init__.py)."""

from .block import DraftBlock
from .draft import KSDraftModel
from .int8_convert import int8_surfaces, to_int8
from .ks3 import KS3, spine_horner
from .rosa import RosaMixer, _match_payload_sign
from .spine import AdjacentInjection

__all__ = ["KS3", "spine_horner", "RosaMixer", "AdjacentInjection", "DraftBlock",
           "KSDraftModel", "to_int8", "int8_surfaces", "_match_payload_sign"]
