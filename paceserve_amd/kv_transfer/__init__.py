"""KV-cache migration: the reference's kv_transfer interface over HIP kernels."""

from .kv_utils import KVhelper  # noqa: F401
