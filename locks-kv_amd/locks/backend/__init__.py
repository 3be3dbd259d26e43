"""Engine integration: plugin registration and the hot-path runtime glue."""
