"""Alias: this module is ``sinkattn_amd.pooling_kernel``."""
import sys

import sinkattn_amd.pooling_kernel as _impl

sys.modules[__name__] = _impl
