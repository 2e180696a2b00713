"""The oracle: a CPU restatement of squirrel-rs's Llama token loop.

TEST INFRASTRUCTURE ONLY.  Only tests/, the smoke() entry point and the
bench's cpu_baseline leg may import it; the product never does.
"""
