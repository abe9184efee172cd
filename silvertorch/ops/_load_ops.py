"""``import silvertorch.ops._load_ops`` registers torch.ops.st.* from this
build's HIP extension (silvertorch_amd.ops._load_ops), with the same
no-fallback rule: a missing extension raises ImportError."""

import silvertorch_amd.ops._load_ops  # noqa: F401
