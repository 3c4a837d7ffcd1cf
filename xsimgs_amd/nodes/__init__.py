"""Scene-assembly nodes that feed the rasterization path (reference src/xsimgs/nodes: container)."""
from .container import (RigidTransformAndPut, packed_mask_from_instances, rigid_transform_and_put,
                        rigid_transform_and_put_torch)

__all__ = ["RigidTransformAndPut", "rigid_transform_and_put", "rigid_transform_and_put_torch",
           "packed_mask_from_instances"]
