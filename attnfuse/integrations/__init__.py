"""``attnfuse.integrations`` -- see ``attentionfuse_amd.integrations``."""
