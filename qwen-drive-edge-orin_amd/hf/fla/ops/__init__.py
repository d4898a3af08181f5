"""See ``fla/__init__.py``: only ``ops.gated_delta_rule`` is provided."""

from . import gated_delta_rule  # noqa: E402,F401
