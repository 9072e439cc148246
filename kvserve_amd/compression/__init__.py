"""Drop-in mirror of kvserve_v1.compression for the MI355X engine."""
