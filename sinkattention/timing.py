"""Alias: this module is ``sinkattn_amd.timing``."""
import sys

import sinkattn_amd.timing as _impl

sys.modules[__name__] = _impl
