"""Per-op modules mirroring the reference's kernel files (descriptor, config
list, build function) on top of the AOT gfx950 instances."""
