"""CPU oracle for the W4A16 path. Test infrastructure only: imported by tests/, smoke() and the
cpu_baseline leg of bench.py, never by the product."""
