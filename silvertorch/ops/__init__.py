"""``silvertorch.ops``: see silvertorch_amd.ops."""
