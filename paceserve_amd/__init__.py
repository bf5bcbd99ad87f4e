"""MI355X-native KV-cache migration path of PaceServe.

paceserve_amd.kv_transfer.kv_utils.KVhelper is a drop-in for
paceserve.kv_transfer.kv_utils.KVhelper; its page movement runs in hand-written
HIP kernels for gfx950 (libpace_kv.so, C ABI in include/pace_kv.h).
"""

__version__ = "0.1.0"
