"""Native-library binding, ABI structs and gradient destinations."""
