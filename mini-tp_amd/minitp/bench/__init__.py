"""Measurement helpers with the reference's timing windows (minitp/bench)."""
