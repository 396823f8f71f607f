"""Error taxonomy and global configuration shared by the host-side modules."""
