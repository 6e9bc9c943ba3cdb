"""Route n-gram memory modules with the reference's names, signatures and state_dict keys.

Forward passes run on hand-written gfx950 kernels (``lngram_hip``); tensors must live
on a ROCm device.  Construction and ``state_dict`` handling work anywhere.
"""
