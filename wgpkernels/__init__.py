"""Import name of the reference package: callers written for WGPKernels (`from wgpkernels import int8 as wq`,
`import wgpkernels.int8`) get this build's MI355X INT8 linear, wgpkernels_amd.int8, unchanged. Only the int8 family
exists in this build."""
import sys

from wgpkernels_amd import int8

sys.modules[__name__ + ".int8"] = int8
__all__ = ["int8"]
