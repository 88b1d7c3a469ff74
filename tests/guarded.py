"""Guarded device buffers for memory-discipline tests: a tensor of numel elements sits at byte
offset GUARD inside a larger allocation whose bytes all start as 255 (NaN for fp16, bf16 and
fp32); intact() reports whether the guard regions before and after it still hold that."""
GUARD = 4096   # bytes on each side (a multiple of 256, so the tensor keeps its alignment)


class Guarded:
    def __init__(self, numel, dtype, device):
        import torch
        esz = torch.empty(0, dtype=dtype).element_size()
        self.nbytes = numel * esz
        self.raw = torch.full((GUARD * 2 + self.nbytes,), 255, dtype=torch.uint8, device=device)
        self.t = self.raw[GUARD:GUARD + self.nbytes].view(dtype)

    def intact(self):
        import torch
        g = torch.cat([self.raw[:GUARD], self.raw[GUARD + self.nbytes:]])
        return bool((g == 255).all())


def from_numpy16(bits, dtype_name):
    """A flat host tensor of 16-bit values (uint16 bit patterns) as torch fp16 / bf16."""
    import numpy as np
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).reshape(-1))
    return t.view(torch.float16 if dtype_name == "f16" else torch.bfloat16)
