"""MI355X (gfx950) implementation of ShardCompute's per-rank quantized inference path.

* ``shardcompute_amd.parallel`` — drop-in layer classes with the reference's
  constructor / forward signatures (quantized column/row linears, embeddings,
  attention, MLP, transformer) at world_size 1 or one rank's shard.
* ``shardcompute_amd._lib`` — ctypes binding of ``libshardcompute_hip.so``, the
  C-ABI declared in ``include/shardcompute_hip.h``.
* ``shardcompute_amd.build`` — hipcc build of that library for gfx950.
"""
__version__ = "0.1.0"
