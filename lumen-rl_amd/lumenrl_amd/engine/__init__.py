"""Engine-side entry points (lumenrl/engine mirror): the weight loader."""
