"""Graph builders for the reference's examples and the five benchmark configs."""
