"""Alias: this module is ``sinkattn_amd.sparse_attention``."""
import sys

import sinkattn_amd.sparse_attention as _impl

sys.modules[__name__] = _impl
