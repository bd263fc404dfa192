"""Plan build, policy loading and the host planning API."""
