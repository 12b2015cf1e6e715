"""Run / compare / measure entry points of the MI355X decode path (the reference's harness/)."""
