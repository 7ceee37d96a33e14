from .foreach import group_tensors_by_shape, move_tensors_to_device

__all__ = ["group_tensors_by_shape", "move_tensors_to_device"]
