"""A<->F transport: arena layout, doorbells, one-GPU channel and server."""
