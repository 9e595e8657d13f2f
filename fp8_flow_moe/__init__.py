"""Drop-in module name for nanopsyche: ``from fp8_flow_moe import ...``
(reference fp8/__init__.py:8-22) resolves to the MI355X implementation in
``nanopysche_amd``."""

from nanopysche_amd import *  # noqa: F401,F403
from nanopysche_amd import __all__  # noqa: F401
