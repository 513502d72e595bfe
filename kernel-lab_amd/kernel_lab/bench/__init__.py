"""Benchmarks and roofline bookkeeping: ``python -m kernel_lab.bench --help`` (needs an MI355X)."""
