"""MI355X-native Mixture-of-Experts layer (forward + backward) for oxidizr."""
