"""Single-rank communicator: the collectives of one GPU's shard.

The reference's ``Communicator`` (``src/shardcompute/collectives/communicator.py:259-561``)
moves tensors between ranks over TCP.  On one GPU every collective of a
world_size = 1 group is the identity, and a rank's shard measured on its own
keeps its partial result (the all-reduce replaced by identity).  The methods
keep the reference's awaitable signatures so the layer code is unchanged.
"""


class IdentityCommunicator:
    def __init__(self, rank: int = 0, world_size: int = 1):
        self.rank = rank
        self.world_size = world_size
        self.calls = {"all_reduce": 0, "all_gather": 0, "broadcast": 0, "barrier": 0}

    async def all_reduce(self, tensor, op: str = "sum"):
        if op not in ("sum", "mean", "max", "min"):
            raise ValueError(f"unsupported reduce op {op}")
        self.calls["all_reduce"] += 1
        return tensor

    async def all_gather(self, tensor, dim: int = -1):
        self.calls["all_gather"] += 1
        return tensor

    async def broadcast(self, tensor, root: int = 0):
        self.calls["broadcast"] += 1
        return tensor

    async def barrier(self):
        self.calls["barrier"] += 1
