"""Host side of the MI355X decode path: the plan (graph_plan), the packed seeded weights
(pack_weights), the task-table builder (build_graph) and the ctypes runtime (runtime)."""
