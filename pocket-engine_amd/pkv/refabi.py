"""Loads pkv_kernels.hsaco and launches its kernels the way the reference
engine does: hipModuleLoadData + hipModuleGetFunction by name
(src/gpu.rs:434-466, 552-566) and hipModuleLaunchKernel with an array of up
to 32 eight-byte argument slots, pointers as u64 and 4-byte values at the
start of their slot (src/gpu.rs:903-930). The launch shapes are the
reference host's (src/model.rs:23-46, 58-141, 2366-2493), restated here so a
test reads like the reference's own call sites.
"""
import ctypes
import os

import torch  # noqa: F401  (the HIP runtime this process already uses)

# PKV_KERNELS selects another build of the code object, as POCKET_KERNELS
# does for the reference engine (src/gpu.rs:451-457).
HSACO = os.environ.get("PKV_KERNELS") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                      "pkv_kernels.hsaco")
HEAD_DIM = 256
SPLIT_MIN_KEYS = 64   # model.rs:26 (ROCm)
SPLIT_MAX = 64        # model.rs:38


def split_ranges(t, hkv, sms):
    """Key ranges per decode token (model.rs:43-46)."""
    return max(1, min(SPLIT_MAX, -(-(4 * sms) // (t * hkv))))


def flash_launch(t, s, hkv, g=4, mfma=False, fp8=False):
    """(name, grid, threads, dynamic smem) of the prompt kernel as fa_shape
    picks it (model.rs:58-79, 112-141, 2455-2463) for a gfx950 device
    (compute capability 9.5): a bf16 cache takes attn_groupr_g4_t2_k32 or
    attn_groupr_g6_t1_k32 (queries in registers, 32-key tiles), other groups
    and every E4M3 cache the 16-key default attn_group[8]_g<G>_t<NT>_k16 with
    NT = 1 for G = 6, else 8 / G; mfma: gfx942's attn_mfma_g<G>_t2."""
    if mfma and not fp8:
        tiles, keys = 2, 32
        name, threads = f"attn_mfma_g{g}_t{tiles}", 64 * g * tiles
        smem = (keys * (HEAD_DIM + 8) + HEAD_DIM * (keys + 8)) * 2
    elif not fp8 and g in (4, 6):
        tiles, keys = (2 if g == 4 else 1), 32
        name, threads = f"attn_groupr_g{g}_t{tiles}_k{keys}", 32 * g * tiles
        smem = max(g * 16 * tiles, 4 * keys) * (HEAD_DIM + 8) * 2
    else:
        tiles, keys = (1 if g == 6 else 8 // g), 16
        name, threads = f"attn_group{'8' if fp8 else ''}_g{g}_t{tiles}_k{keys}", 32 * g * tiles
        smem = (g * 16 * tiles + 4 * keys) * (HEAD_DIM + 8) * 2
    return name, (-(-t // (16 * tiles)) + s, hkv, 1), threads, smem


class P:
    """Pointer argument (a torch tensor, an int address or None); keeps the
    tensor alive as long as the argument list."""

    def __init__(self, v):
        self.keep = v
        self.v = 0 if v is None else (v if isinstance(v, int) else v.data_ptr())


class I:
    def __init__(self, v):
        self.v = int(v) & 0xFFFFFFFF


class F:
    def __init__(self, v):
        self.v = ctypes.c_uint32.from_buffer(ctypes.c_float(v)).value


class RefKernels:
    def __init__(self, path=HSACO):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built (python pocket-engine_amd/build.py)")
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipModuleLoadData.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p]
        self.hip.hipModuleGetFunction.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_char_p]
        self.hip.hipModuleLaunchKernel.argtypes = [ctypes.c_void_p] + [ctypes.c_uint] * 7 + [
            ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p]
        self.image = open(path, "rb").read()
        self.mod = ctypes.c_void_p()
        self._check(self.hip.hipModuleLoadData(ctypes.byref(self.mod), self.image), "hipModuleLoadData")
        self.funcs = {}

    def _check(self, r, what):
        if r != 0:
            raise RuntimeError(f"{what} failed: hip error {r}")

    def kernel(self, name):
        if name not in self.funcs:
            f = ctypes.c_void_p()
            self._check(self.hip.hipModuleGetFunction(ctypes.byref(f), self.mod, name.encode()),
                        f"hipModuleGetFunction({name})")
            self.funcs[name] = f
        return self.funcs[name]

    def launch(self, name, grid, block, smem, args, stream=None):
        assert len(args) <= 32
        vals = (ctypes.c_uint64 * 32)()
        for i, a in enumerate(args):
            vals[i] = a.v
        ptrs = (ctypes.c_void_p * 32)()
        for i in range(len(args)):
            ptrs[i] = ctypes.addressof(vals) + 8 * i
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        self._check(self.hip.hipModuleLaunchKernel(self.kernel(name), grid[0], grid[1], grid[2], block, 1, 1, smem, s,
                                                   ptrs, None), f"hipModuleLaunchKernel({name})")
