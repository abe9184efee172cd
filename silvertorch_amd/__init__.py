"""MI355X-native bloom-index retrieval path (torch.ops.st.* drop-in).

``import silvertorch_amd.ops._load_ops`` registers torch.ops.st.* from the
in-tree HIP extension; see include/silvertorch_hip.h for the C ABI beneath it.
"""

__version__ = "0.1.0"
