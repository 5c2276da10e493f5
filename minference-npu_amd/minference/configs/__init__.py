"""Pattern configs: the MODEL2PATH registry and the seeded pattern generator."""
