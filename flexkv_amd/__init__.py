"""flexkv_amd: MI355X (gfx950) GPU<->CPU KV-block transfer for FlexKV.

Drop-in modules for the reference's transfer path:
  flexkv_amd.c_ext               <- flexkv.c_ext.transfer_kv_blocks
  flexkv_amd.transfer.worker     <- flexkv.transfer.worker (GPU<->CPU worker)
  flexkv_amd.common.storage      <- flexkv.common.storage (KVCacheLayout)
  flexkv_amd.common.transfer     <- flexkv.common.transfer (TransferOp, ...)
  flexkv_amd.common.config       <- flexkv.common.config (hot-path knobs)
  flexkv_amd.common.memory_handle<- flexkv.common.memory_handle
  flexkv_amd.storage.allocator   <- flexkv.storage.allocator (CPU/GPU)
"""
__version__ = "0.1.0"
