"""Engine, workspace and hipGraph lifecycle."""
