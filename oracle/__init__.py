"""ORACLE — CPU restatement of the reference's native-CPU path, used only by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker / CPU baseline."""
